// Storage handles and the drop-in Backend trait (orca-tensor/src/backend.rs:7-315)
// over the buffer-level entry points of liborca_hip.so.
//
// A backend (orca_hip_backend) owns the planning state that makes the composed
// training step cheap without the tape noticing: lazy transpose views, pending
// elementwise chains run as one fused program, pending products run with their
// epilogue, the deferred bias column sum and the identity-reduction memo,
// one-element host constants, and the events of the fused optimizer's
// second-stream pass.  A storage (orca_hip_storage) is a reference-counted node:
// either a computed value (a device buffer, possibly a transposed view of one),
// or a pending op over other nodes.
//
// Whether an intermediate of a pending chain is written out is decided from
// reference counts: a node referenced beyond the links inside the chain being run
// (a binding's handle, a tape's saved primal, another pending op) is written by
// the same launch.  Every value has the bits the trait's ops run one by one give:
// each fused instruction and each folded epilogue is the op's own f32 operation.
//
// This file launches nothing itself: it calls the library's buffer-level entry
// points, so it also builds on the CPU against a stand-in of them (tests/native).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <map>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "runtime.hpp"

namespace orca_hip {
namespace {

// Rethrows the failure of a nested entry point with its code and fields.
void ck(int rc) {
  if (rc == ORCA_HIP_OK) return;
  orca_hip_error_info info{};
  last_error_info(&info);
  ErrorFields f;
  f.op = info.op ? info.op : "";
  f.expected = info.expected ? info.expected : "";
  f.got = info.got ? info.got : "";
  f.dtype = info.dtype;
  f.dtype_got = info.dtype_got;
  for (int i = 0; i < 2; ++i) {
    f.device_kind[i] = info.device_kind[i];
    f.device_index[i] = info.device_index[i];
  }
  throw Error(rc, info.message ? info.message : "", std::move(f));
}

// The guard of this file's entry points: like guard(), but the buffers that nested
// entry points return are owned by nodes here, so a failure must not release them
// again (each nested call commits its own outputs).
template <class F>
int guard_nodes(F&& f) {
  try {
    f();
    return ORCA_HIP_OK;
  } catch (const Error& e) {
    set_last_error(e.what(), e.code, e.fields);
    return e.code;
  } catch (const std::exception& e) {
    set_last_error(std::string("internal error: ") + e.what());
    return ORCA_HIP_ERR_INTERNAL;
  } catch (...) {
    set_last_error("internal error: unknown exception");
    return ORCA_HIP_ERR_INTERNAL;
  }
}

size_t numel_of(const size_t* shape, size_t rank) {
  size_t n = 1;
  for (size_t i = 0; i < rank; ++i) n *= shape[i];
  return n;
}

// ------------------------------------------------------------------ nodes
// Device memory of computed values.  A view (an arena slice) keeps its arena alive
// and frees nothing itself.
struct Buf {
  orca_hip_ctx* ctx = nullptr;
  float* ptr = nullptr;
  size_t bytes = 0;
  std::shared_ptr<Buf> owner;
  ~Buf() {
    if (!owner && ptr) (void)orca_hip_free(ctx, ptr);
  }
};
using BufP = std::shared_ptr<Buf>;

struct Planner;
using Backend = Planner;
struct Node;

// A point in one stream's work (an event) that orders the context's two streams.
// `keep` holds what the work before it reads, until the context stream has been
// made to wait for it, so their blocks are not reused before that work is done.
struct Mark {
  Backend* be = nullptr;
  orca_hip_event* ev = nullptr;
  uint64_t seq = 0;
  // the allocator's release clock when the mark was recorded: blocks released by then
  // were last used by work before it
  uint64_t clock = 0;
  std::vector<Node*> keep;
  bool settled = false;
  ~Mark();
};
using MarkP = std::shared_ptr<Mark>;

enum class Kind : uint8_t {
  kValue,   // computed: buf (null only for a folded product nobody reads)
  kEw,      // pending elementwise op over operand nodes
  kProd,    // pending 2-D product lhs x rhs
  kColsum,  // pending sum_to_shape(src [rows, cols] -> [1, cols])
  kConst,   // one-element value known on the host, not yet on the device
  kBcast,   // an elementwise program input: src read as src[(e / div) % mod] (Backend::expand)
};

struct Node {
  std::atomic<int> rc{1};
  Backend* be = nullptr;
  size_t n = 0;
  Kind kind = Kind::kValue;
  BufP buf;
  // A lazy last-two-dims transpose of a computed value: its logical shape (the
  // buffer holds the untransposed data); empty for contiguous storage.
  std::vector<size_t> tshape;
  // kEw: opcode, operands (held), scalar, and upper bounds of the ops and distinct
  // inputs of its pending chain
  uint8_t op = 0, nopd = 0;
  Node* opd[3] = {nullptr, nullptr, nullptr};
  float scalar = 0.0f;
  int ew_ops = 0, ew_leaves = 1;
  // kProd: operands (held), dims and views; kColsum / kBcast: src (held) in lhs
  Node* lhs = nullptr;
  Node* rhs = nullptr;
  size_t M = 0, K = 0, N = 0;
  bool lt = false, rt = false;
  // A pending weight gradient X^T G whose bias gradient (a pending column sum of G) it computes
  // (held); and, on that column sum, the product that will (weak).
  Node* cs = nullptr;
  Node* via = nullptr;
  uint64_t div = 1, mod = 1;  // kBcast
  // a one-element value known on the host (kConst, and after its upload)
  bool has_const = false;
  float cval = 0.0f;
  // This node's identity sum_to_shape result, and its source (weak links, cleared
  // by whichever dies first).
  Node* ident = nullptr;
  Node* ident_of = nullptr;
  // Pending column sums of this node (weak; each clears its entry when it dies or runs).
  std::vector<Node*> waiters;
  // Written on the second stream: the mark its first use waits for on the context stream.
  MarkP ready;
  // Made by a weight-gradient product: the mark just after that launch.
  MarkP made;
  // The mark count when the value was computed on the context stream: the context stream's
  // marks with a higher count come after that work.
  uint64_t done_seq = 0;
  // Computed on the second stream (later work there is ordered after it).
  bool side_made = false;
  // Written in place by an update after it was computed (never read on the second stream).
  bool in_place = false;
  // Computed by arithmetic (a product, a loss): it holds no signaling NaN, so x * 1 is x.
  bool quiet = false;
  // Holds no -0 either (a loss gradient whose every element is a sum of terms that are never
  // -0), so 0 + x is x too: its identity sum_to_shape is the value itself.
  bool canon = false;
  bool in_pending = false;
  uint64_t pseq = 0;  // creation order among pending nodes

  bool pending() const {
    return kind == Kind::kEw || kind == Kind::kProd || kind == Kind::kColsum || kind == Kind::kConst;
  }
};

// A compiled elementwise program (register allocation and instructions) of one
// chain structure; the chain's scalars are written into it before each launch.
struct Program {
  bool ok = false;
  std::vector<orca_hip_ew_instr> instrs;
  std::vector<uint8_t> oregs;
  size_t n_regs = 0;
  std::vector<int> scalar_at;
};

// The planning state of one context, shared by every backend handle on it (so storages
// pass freely between handles with different switches on one context).
struct Planner {
  std::atomic<int> rc{1};  // one per backend handle plus one per live node
  orca_hip_ctx* ctx = nullptr;
  std::mutex mu;
  // the switches of the handle whose call is running (set at each entry, under mu)
  orca_hip_backend_options opt{};
  // Backward products leave marks once a fused optimizer pass has asked for them (the
  // last few kept: the pass splits its side-stream part at the one before the last).
  bool marking = false;
  std::deque<MarkP> recent;
  uint64_t mark_seq = 0;
  bool on_side = false;
  // the weight or bias gradient that an elementwise op read last (an address, never followed)
  const Node* grad_read = nullptr;
  // nodes created with a pending elementwise op or product and not yet computed, in
  // creation order
  std::map<uint64_t, Node*> pending;
  uint64_t pending_seq = 0;
  std::unordered_map<std::string, Program> programs;
  // nodes whose last reference went while one was being destroyed (drained in a loop)
  std::vector<Node*> dying;
  bool draining = false;
};

}  // namespace
}  // namespace orca_hip

// A backend handle: the context's planner and this handle's switches.
struct orca_hip_backend {
  orca_hip::Planner* pl = nullptr;
  orca_hip_backend_options opt{};
};

namespace orca_hip {
namespace {

inline Node* N_(orca_hip_storage* s) { return reinterpret_cast<Node*>(s); }
inline orca_hip_storage* S_(Node* n) { return reinterpret_cast<orca_hip_storage*>(n); }

// Planners by context.
std::mutex g_planners_mu;
std::map<orca_hip_ctx*, Planner*>& planners() {
  static std::map<orca_hip_ctx*, Planner*> m;
  return m;
}

// Drops a reference to a planner; never called with its lock held when it may be the last.
void backend_unref(Backend* be) {
  std::lock_guard<std::mutex> lk(g_planners_mu);
  if (be->rc.fetch_sub(1, std::memory_order_acq_rel) == 1) {
    auto& m = planners();
    auto it = m.find(be->ctx);
    if (it != m.end() && it->second == be) m.erase(it);
    delete be;
  }
}

Planner* planner_for(orca_hip_ctx* ctx) {
  std::lock_guard<std::mutex> lk(g_planners_mu);
  auto& m = planners();
  auto it = m.find(ctx);
  if (it != m.end()) {
    it->second->rc.fetch_add(1, std::memory_order_relaxed);
    return it->second;
  }
  auto* pl = new Planner();
  pl->ctx = ctx;
  m[ctx] = pl;
  return pl;
}

void destroy_node(Node* x);

// Drops one reference (the backend lock is held).  Destruction cascades through
// operands iteratively.
void unref(Node* x) {
  if (!x) return;
  if (x->rc.fetch_sub(1, std::memory_order_acq_rel) != 1) return;
  Backend* be = x->be;
  be->dying.push_back(x);
  if (be->draining) return;
  be->draining = true;
  while (!be->dying.empty()) {
    Node* d = be->dying.back();
    be->dying.pop_back();
    destroy_node(d);
  }
  be->draining = false;
}

inline Node* ref(Node* x) {
  x->rc.fetch_add(1, std::memory_order_relaxed);
  return x;
}

// An owning pointer for temporaries.
struct Ref {
  Node* p = nullptr;
  Ref() = default;
  explicit Ref(Node* q) : p(q) {}  // adopts a reference
  Ref(const Ref&) = delete;
  Ref(Ref&& o) noexcept : p(o.p) { o.p = nullptr; }
  Ref& operator=(Ref&& o) noexcept {
    if (this != &o) {
      unref(p);
      p = o.p;
      o.p = nullptr;
    }
    return *this;
  }
  ~Ref() { unref(p); }
  Node* get() const { return p; }
  Node* operator->() const { return p; }
  Node* release() {
    Node* q = p;
    p = nullptr;
    return q;
  }
};

Node* new_node(Backend* be, size_t n) {
  Node* x = new Node();
  x->be = be;
  x->n = n;
  be->rc.fetch_add(1, std::memory_order_relaxed);
  return x;
}

Node* value_node(Backend* be, size_t n, BufP buf) {
  Node* x = new_node(be, n);
  x->buf = std::move(buf);
  x->done_seq = be->mark_seq;
  return x;
}

BufP own(orca_hip_ctx* ctx, void* p, size_t bytes) {
  auto b = std::make_shared<Buf>();
  b->ctx = ctx;
  b->ptr = static_cast<float*>(p);
  b->bytes = bytes;
  return b;
}

BufP alloc_buf(Backend* be, size_t n) {
  void* p = nullptr;
  ck(orca_hip_alloc(be->ctx, 4 * std::max<size_t>(n, 1), &p));
  return own(be->ctx, p, 4 * std::max<size_t>(n, 1));
}

void drop_operands(Node* x) {
  for (int i = 0; i < x->nopd; ++i) {
    Node* o = x->opd[i];
    x->opd[i] = nullptr;
    unref(o);
  }
  x->nopd = 0;
  Node* l = x->lhs;
  Node* r = x->rhs;
  x->lhs = x->rhs = nullptr;
  unref(l);
  unref(r);
  if (Node* c = x->cs) {
    x->cs = nullptr;
    c->via = nullptr;
    unref(c);
  }
}

void unwait(Node* colsum_node) {  // removes a pending column sum from its source's waiters
  Node* src = colsum_node->lhs;
  if (!src) return;
  auto& w = src->waiters;
  w.erase(std::remove(w.begin(), w.end(), colsum_node), w.end());
}

// The node becomes a computed value.
void set_value(Node* x, BufP buf) {
  Backend* be = x->be;
  if (x->kind == Kind::kColsum) unwait(x);
  x->buf = std::move(buf);
  x->kind = Kind::kValue;
  x->done_seq = be->mark_seq;
  x->ew_ops = 0;
  x->ew_leaves = 1;
  if (x->in_pending) {
    be->pending.erase(x->pseq);
    x->in_pending = false;
  }
  drop_operands(x);
}

void destroy_node(Node* x) {
  Backend* be = x->be;
  if (x->in_pending) be->pending.erase(x->pseq);
  if (x->kind == Kind::kColsum) unwait(x);
  for (Node* w : x->waiters) w->lhs = nullptr;  // cannot happen while a waiter holds x; kept for safety
  x->waiters.clear();
  if (x->ident) x->ident->ident_of = nullptr;
  if (x->ident_of) x->ident_of->ident = nullptr;
  drop_operands(x);
  if (x->ready && !x->ready->settled && x->buf && !be->on_side) {
    // written on the second stream and never used on the context stream: that stream
    // waits for the write before the block can go back to the allocator
    (void)orca_hip_event_wait(be->ctx, x->ready->ev);
  }
  x->ready.reset();
  x->made.reset();
  x->buf.reset();
  delete x;
  backend_unref(be);
}

Mark::~Mark() {
  if (!keep.empty() && !settled && be && be->ctx) {
    // the context stream waits for the mark before the kept blocks can be reused
    (void)orca_hip_event_wait(be->ctx, ev);
  }
  for (Node* k : keep) unref(k);
  if (be && be->ctx && ev) (void)orca_hip_event_release(be->ctx, ev);
}

// A mark on the current stream: `ev` when given (an event a launch records itself), else an
// event recorded now.
MarkP new_mark(Backend* be, orca_hip_event* ev = nullptr) {
  auto m = std::make_shared<Mark>();
  m->be = be;
  if (ev) {
    m->ev = ev;
  } else {
    ck(orca_hip_event_record(be->ctx, &m->ev));
  }
  m->seq = ++be->mark_seq;
  m->clock = ctx_release_clock(be->ctx);
  return m;
}

// A backward product's mark on the context stream, kept among the recent ones.
MarkP record_mark(Backend* be, orca_hip_event* ev = nullptr) {
  MarkP m = new_mark(be, ev);
  be->recent.push_back(m);
  while (be->recent.size() > 8) be->recent.pop_front();
  return m;
}

// Whether backward products leave marks: with the second stream allowed, or once a fused
// optimizer pass has asked for them.
bool marking(Backend* be) { return be->marking || be->opt.overlap; }

// The context stream waits for the mark (once); the kept storages can go.
void settle(Backend* be, Mark& m) {
  if (be->on_side) fail(ORCA_HIP_ERR_INTERNAL, "a marked storage was used while launches go to the second stream");
  if (!m.settled) {
    m.settled = true;
    ck(orca_hip_event_wait(be->ctx, m.ev));
    std::vector<Node*> keep;
    keep.swap(m.keep);
    for (Node* k : keep) unref(k);
  }
}

// ------------------------------------------------------------------ computing values
void flush(Backend* be, Node* root);
void run_product(Backend* be, Node* x);
struct Buf;
Buf* materialize(Backend* be, Node* x);

void track_pending(Backend* be, Node* x) {
  x->in_pending = true;
  x->pseq = ++be->pending_seq;
  be->pending.emplace(x->pseq, x);
}

// Computes every pending value, in creation order (a backward pass's order).
void flush_all(Backend* be) {
  while (!be->pending.empty()) {
    Ref x(ref(be->pending.begin()->second));
    materialize(be, x.get());
    if (x->in_pending) fail(ORCA_HIP_ERR_INTERNAL, "a pending storage stayed pending when computed");
  }
}


// The node's values on the device (computing what is pending); the buffer.  A value written
// on the second stream (before, or by computing it just now) is waited for first.
Buf* materialize(Backend* be, Node* x) {
  switch (x->kind) {
    case Kind::kEw:
      flush(be, x);
      break;
    case Kind::kProd:
      run_product(be, x);
      break;
    case Kind::kColsum: {
      if (x->via) {  // the weight gradient that computes it as well
        Ref v(ref(x->via));
        materialize(be, v.get());
        if (x->kind == Kind::kValue) break;
      }
      Ref src(ref(x->lhs));
      Buf* sb = materialize(be, src.get());
      const size_t in_shape[2] = {x->M, x->N}, out_shape[2] = {1, x->N};
      void* out = nullptr;
      ck(orca_hip_sum_to_shape(be->ctx, sb->ptr, in_shape, 2, out_shape, 2, ORCA_HIP_F32, &out));
      set_value(x, own(be->ctx, out, 4 * std::max<size_t>(x->N, 1)));
      break;
    }
    case Kind::kConst: {
      const size_t shape[1] = {1};
      void* out = nullptr;
      ck(orca_hip_from_f32_slice(be->ctx, shape, 1, &x->cval, 1, &out));
      set_value(x, own(be->ctx, out, 4));
      break;
    }
    case Kind::kBcast:
      fail(ORCA_HIP_ERR_INTERNAL, "a broadcast input has no buffer of its own");
    case Kind::kValue:
      break;
  }
  if (x->ready) {
    MarkP m = std::move(x->ready);
    settle(be, *m);
  }
  if (!x->buf) fail(ORCA_HIP_ERR_INTERNAL, "storage has no values (a product folded into its epilogue)");
  return x->buf.get();
}

float* dptr(Backend* be, Node* x) { return materialize(be, x)->ptr; }

// A contiguous node with x's logical values: x itself, or the materialised transpose of a view.
Ref plain(Backend* be, Node* x) {
  if (x->tshape.empty()) return Ref(ref(x));
  std::vector<size_t> src_shape = x->tshape;
  const size_t r = src_shape.size();
  std::swap(src_shape[r - 1], src_shape[r - 2]);
  float* p = dptr(be, x);
  void* out = nullptr;
  ck(orca_hip_transpose(be->ctx, p, src_shape.data(), r, r - 2, r - 1, ORCA_HIP_F32, &out));
  return Ref(value_node(be, x->n, own(be->ctx, out, 4 * std::max<size_t>(x->n, 1))));
}

// The pending weight gradient H^T G (with its bias gradient) beside the narrow product
// p = G W^T (a classifier head's backward, K <= 16), or null.
Node* narrow_sibling(Node* p) {
  if (!p || p->kind != Kind::kProd || p->lt || !p->rt || p->K > 16) return nullptr;
  Node* g = p->lhs;
  for (Node* t : g->waiters) {
    Node* x = t->kind == Kind::kColsum ? t->via : nullptr;
    if (x && x->kind == Kind::kProd && x->cs == t && x->rhs == g && x->lt && !x->lhs->tshape.empty() &&
        x->M == p->N && x->K == p->M && x->N == p->K)
      return x;
  }
  return nullptr;
}

// p = G W^T (into c, through the ReLU mask of `mask_node` when given, with the unmasked
// product into `pre` when given), its sibling weight gradient x = H^T G and x's bias gradient
// from one grid (orca_hip_narrow_linear_backward: the same sums as the three run one by one).
// Sets x and its bias gradient; the caller sets p and the epilogue's outputs.
void run_narrow_backward(Backend* be, Node* p, Node* x, Node* mask_node, float* c, float* pre) {
  Ref px(ref(p)), xx(ref(x)), tt(ref(x->cs));
  Node* target = tt.get();
  float* hp = dptr(be, x->lhs);  // H's own buffer (H^T is a view of it)
  float* gp = dptr(be, p->lhs);
  float* wp = dptr(be, p->rhs);  // W's own buffer (W^T is a view of it)
  float* mp = mask_node ? dptr(be, mask_node) : nullptr;
  const size_t B = p->M, K = p->N, C = p->K;
  BufP dw = alloc_buf(be, K * C), db = alloc_buf(be, C);
  const bool mark = marking(be);
  orca_hip_event* ev = nullptr;
  ck(orca_hip_narrow_linear_backward(be->ctx, hp, B, K, gp, C, wp, mp, c, pre, dw->ptr, db->ptr, mark ? &ev : nullptr));
  set_value(target, db);
  set_value(x, dw);
  if (mark) {
    MarkP m = record_mark(be, ev);
    x->made = target->made = m;  // a weight gradient and its bias gradient
  }
}

void run_product(Backend* be, Node* x) {
  if (Node* w = narrow_sibling(x)) {  // a head's input gradient, with the weight gradient beside it
    BufP c = alloc_buf(be, x->M * x->N);
    run_narrow_backward(be, x, w, nullptr, c->ptr, nullptr);
    set_value(x, c);
    return;
  }
  Ref lhs(ref(x->lhs)), rhs(ref(x->rhs));
  const size_t M = x->M, K = x->K, N = x->N;
  const bool lt = x->lt, rt = x->rt;
  float* a = dptr(be, lhs.get());
  float* b = dptr(be, rhs.get());
  const bool mark = marking(be) && (lt || rt);  // a backward product
  if (x->cs) {  // a weight gradient run alone, with its bias gradient in the same launch
    Ref tt(ref(x->cs));
    Node* target = tt.get();
    BufP cs = alloc_buf(be, N);
    void* out = nullptr;
    orca_hip_event* ev = nullptr;
    ck(orca_hip_matmul_ev(be->ctx, a, b, M, K, N, ORCA_HIP_VIEW_TRANSPOSED, ORCA_HIP_VIEW_CONTIGUOUS, ORCA_HIP_F32,
                          cs->ptr, &out, mark ? &ev : nullptr));
    set_value(target, cs);
    set_value(x, own(be->ctx, out, 4 * M * N));
    if (mark) {
      MarkP m = record_mark(be, ev);
      x->made = target->made = m;
    }
    return;
  }
  void* out = nullptr;
  orca_hip_event* ev = nullptr;
  ck(orca_hip_matmul_ev(be->ctx, a, b, M, K, N, lt ? ORCA_HIP_VIEW_TRANSPOSED : ORCA_HIP_VIEW_CONTIGUOUS,
                        rt ? ORCA_HIP_VIEW_TRANSPOSED : ORCA_HIP_VIEW_CONTIGUOUS, ORCA_HIP_F32, nullptr, &out,
                        mark ? &ev : nullptr));
  set_value(x, own(be->ctx, out, 4 * M * N));
  if (mark) {
    MarkP m = record_mark(be, ev);
    if (lt) x->made = m;  // a weight gradient X^T G
  }
}

// ---- fused elementwise chains
struct Walk {
  std::vector<Node*> order;   // chain ops, post-order (the root last)
  std::vector<Node*> leaves;  // distinct inputs, in first-use order
  std::unordered_map<Node*, int> refmap, inner;
  std::vector<int> sig;       // per op: opcode, operand count, operand refs (leaf i: -1 - i)
  std::vector<int> op_start;  // index of each op's record in sig
  std::vector<float> scalars;

  int visit(Node* node) {
    int refs[3] = {0, 0, 0};
    for (int i = 0; i < node->nopd; ++i) {
      Node* c = node->opd[i];
      auto it = refmap.find(c);
      int r;
      if (c->kind != Kind::kEw) {  // an input
        if (it == refmap.end()) {
          r = -1 - (int)leaves.size();
          refmap[c] = r;
          leaves.push_back(c);
        } else {
          r = it->second;
        }
      } else {
        inner[c] += 1;
        if (it == refmap.end()) {
          r = visit(c);
          refmap[c] = r;
        } else {
          r = it->second;
        }
      }
      refs[i] = r;
    }
    const int k = (int)order.size();
    order.push_back(node);
    op_start.push_back((int)sig.size());
    sig.push_back(node->op);
    sig.push_back(node->nopd);
    for (int i = 0; i < node->nopd; ++i) sig.push_back(refs[i]);
    scalars.push_back(node->scalar);
    return k;
  }
  int op_of(int k) const { return sig[op_start[k]]; }
  int nargs_of(int k) const { return sig[op_start[k] + 1]; }
  int arg_of(int k, int i) const { return sig[op_start[k] + 2 + i]; }
};

// Compiles a chain: inputs take registers 0..n_leaves-1; each op's result takes the
// lowest free register; a register is freed after its value's last use (an output
// keeps its register to the end).  !ok when the interpreter's limits are exceeded.
Program compile(const Walk& w, const std::vector<int>& out_idx) {
  Program p;
  const int n_ops = (int)w.order.size();
  const int n_leaves = (int)w.leaves.size();
  if ((int)out_idx.size() > ORCA_HIP_EW_MAX_OUTPUTS || n_ops > ORCA_HIP_EW_MAX_OPS) return p;
  std::unordered_map<int, int> last;
  for (int k = 0; k < n_ops; ++k)
    for (int i = 0; i < w.nargs_of(k); ++i) last[w.arg_of(k, i)] = k;
  std::unordered_set<int> outs(out_idx.begin(), out_idx.end());
  std::vector<int> free_regs;
  std::vector<int> reg(n_ops, -1);
  int n_regs = n_leaves;
  for (int k = 0; k < n_ops; ++k) {
    const int na = w.nargs_of(k);
    int regs[3];
    for (int i = 0; i < na; ++i) {
      const int r = w.arg_of(k, i);
      regs[i] = r < 0 ? -1 - r : reg[r];
    }
    // free the registers of values whose last use is this op (each distinct ref once)
    for (int i = 0; i < na; ++i) {
      const int r = w.arg_of(k, i);
      bool seen = false;
      for (int j = 0; j < i; ++j) seen = seen || w.arg_of(k, j) == r;
      if (seen) continue;
      if (last[r] == k && (r < 0 || !outs.count(r))) free_regs.push_back(r < 0 ? -1 - r : reg[r]);
    }
    int dst;
    if (!free_regs.empty()) {
      std::sort(free_regs.begin(), free_regs.end());
      dst = free_regs.front();
      free_regs.erase(free_regs.begin());
    } else {
      dst = n_regs++;
    }
    reg[k] = dst;
    for (int i = na; i < 3; ++i) regs[i] = regs[0];
    orca_hip_ew_instr ins{};
    ins.op = (uint8_t)w.op_of(k);
    ins.dst = (uint8_t)dst;
    ins.a = (uint8_t)regs[0];
    ins.b = (uint8_t)regs[1];
    ins.c = (uint8_t)regs[2];
    ins.scalar = 0.0f;
    p.instrs.push_back(ins);
    if (ins.op == ORCA_HIP_EW_MUL_SCALAR || ins.op == ORCA_HIP_EW_ADD_SCALAR) p.scalar_at.push_back(k);
  }
  if (n_regs > ORCA_HIP_EW_MAX_REGS) return p;
  for (int k : out_idx) p.oregs.push_back((uint8_t)reg[k]);
  p.n_regs = (size_t)n_regs;
  p.ok = true;
  return p;
}

// Whether orca_hip_gemm runs the product on its narrow kernels with this epilogue (the GEMM
// planner's rule): a fold is taken only where the plain product and the one with the epilogue
// run on the same kernel, so the same sums.
bool narrow_kernel(int kind, bool lt, bool rt, size_t N, size_t K) {
  if (!lt && !rt && N <= 16) return kind == ORCA_HIP_EPI_NONE || kind == ORCA_HIP_EPI_BIAS;
  if (!lt && rt && K <= 16)
    return kind == ORCA_HIP_EPI_NONE || kind == ORCA_HIP_EPI_RELU_MASK || kind == ORCA_HIP_EPI_RELU_MASK_PRE;
  if (lt && !rt && N <= 16) return kind == ORCA_HIP_EPI_NONE;
  return false;
}

bool sig_is(const Walk& w, std::initializer_list<std::initializer_list<int>> pattern) {
  if (w.order.size() != pattern.size()) return false;
  int k = 0;
  for (auto& rec : pattern) {
    auto it = rec.begin();
    if (w.op_of(k) != *it++) return false;
    if (w.nargs_of(k) != (int)rec.size() - 1) return false;
    for (int i = 0; it != rec.end(); ++it, ++i)
      if (w.arg_of(k, i) != *it) return false;
    ++k;
  }
  return true;
}

// Runs the chain as its product's epilogue when it is one of the forms
//   relu_backward(P, z) [+ its identity sum 0 + x]  (ReluBackward on a product),
//   add(P, expand(b)) [+ relu]                      (Linear's bias, and ReLU),
// over a pending product P (the first input).  A product held beyond the chain's one link
// (a gradient the tape keeps) is written as well by the mask epilogue, and is not folded
// into the bias ones.
bool fold_chain(Backend* be, Walk& w, const std::vector<int>& out_idx, bool shared) {
  Node* prod = w.leaves[0];
  if (prod->kind != Kind::kProd) return false;
  const size_t M = prod->M, K = prod->K, N = prod->N;
  const bool lt = prod->lt, rt = prod->rt;
  using V = std::vector<int>;
  const bool mask = sig_is(w, {{ORCA_HIP_EW_RELU_BW, -1, -2}}) && out_idx == V{0};
  const bool mask_ident = sig_is(w, {{ORCA_HIP_EW_RELU_BW, -1, -2}, {ORCA_HIP_EW_SUM_VISIT, 0}}) &&
                          (out_idx == V{0, 1} || out_idx == V{1});
  const bool bias = sig_is(w, {{ORCA_HIP_EW_COPY, -2}, {ORCA_HIP_EW_ADD, -1, 0}}) && out_idx == V{1};
  const bool bias_relu = sig_is(w, {{ORCA_HIP_EW_COPY, -2}, {ORCA_HIP_EW_ADD, -1, 0}, {ORCA_HIP_EW_RELU, 1}}) &&
                         (out_idx == V{1, 2} || out_idx == V{2});
  int kind;
  Node* bias_src = nullptr;
  Node* mask_node = nullptr;
  if (mask || mask_ident) {
    Node* z = w.leaves[1];
    if (z->kind == Kind::kBcast || !z->tshape.empty() || z->n != M * N) return false;
    kind = shared ? ORCA_HIP_EPI_RELU_MASK_PRE : ORCA_HIP_EPI_RELU_MASK;
    mask_node = z;
  } else if (shared) {
    return false;
  } else if (bias || bias_relu) {
    Node* b = w.leaves[1];
    if (b->kind != Kind::kBcast || b->div != 1 || b->mod != N || b->lhs->n != N || !b->lhs->tshape.empty()) return false;
    kind = bias ? ORCA_HIP_EPI_BIAS : (out_idx == V{1, 2} ? ORCA_HIP_EPI_BIAS_RELU_PRE : ORCA_HIP_EPI_BIAS_RELU);
    bias_src = b->lhs;
  } else {
    return false;
  }
  if (narrow_kernel(kind, lt, rt, N, K) != narrow_kernel(ORCA_HIP_EPI_NONE, lt, rt, N, K)) return false;
  // The operands first: pending work they need is launched before a wait on a mark that a
  // bias or mask written on the second stream brings in.
  Ref lhs(ref(prod->lhs)), rhs(ref(prod->rhs)), pr(ref(prod));
  float* lp = dptr(be, lhs.get());
  float* rp = dptr(be, rhs.get());
  orca_hip_epilogue e{};
  e.kind = kind;
  e.bias = bias_src ? dptr(be, bias_src) : nullptr;
  e.mask = mask_node ? dptr(be, mask_node) : nullptr;
  e.ldmask = mask_node ? N : 0;
  BufP c = alloc_buf(be, M * N);
  BufP pre;
  if (kind == ORCA_HIP_EPI_BIAS_RELU_PRE || kind == ORCA_HIP_EPI_RELU_MASK_PRE) {
    pre = alloc_buf(be, M * N);
    e.pre = pre->ptr;
  }
  Node* wg = mask_node ? narrow_sibling(prod) : nullptr;
  if (wg) {  // a head's input gradient, with the weight gradient beside it
    run_narrow_backward(be, prod, wg, mask_node, c->ptr, pre ? pre->ptr : nullptr);
  } else {
    const bool mark = marking(be) && (lt || rt);  // a backward product
    orca_hip_event* ev = nullptr;
    e.done = mark ? &ev : nullptr;
    ck(orca_hip_gemm(be->ctx, lt ? 1 : 0, rt ? 1 : 0, M, N, K, lp, lt ? M : K, rp, rt ? K : N, c->ptr, N, &e));
    if (mark) record_mark(be, ev);
  }
  if (kind == ORCA_HIP_EPI_RELU_MASK_PRE) {
    set_value(prod, pre);  // the product itself, for its other holders
    pre.reset();
  } else {
    set_value(prod, nullptr);  // nobody else reads it
  }
  std::vector<BufP> outs;
  if (mask_ident) {
    outs.assign(out_idx.size(), c);  // the masked product and its identity sum: one buffer
  } else if (pre) {
    outs = {pre, c};  // out_idx order: the add (pre-activation) before the relu
  } else {
    outs = {c};
  }
  for (size_t i = 0; i < out_idx.size(); ++i) set_value(w.order[out_idx[i]], outs[i]);
  return true;
}

void flush_operands_first(Backend* be, Node* root) {
  Ref keep(ref(root));
  for (int i = 0; i < root->nopd; ++i) {
    Node* c = root->opd[i];
    if (c && c->kind == Kind::kEw) {
      Ref cc(ref(c));
      flush(be, c);
    }
  }
  if (root->kind == Kind::kEw) flush(be, root);
}

// Runs a chain on the context's second stream, beside the products launched after its
// inputs, when the second stream is allowed, every input is computed and such a product
// exists (an optimizer update whose gradient came before the backward's last products).
// The program waits for the first context-stream mark after its inputs were computed there
// (inputs written on the second stream are ordered there already); its outputs take cached
// blocks released before that mark, so no context-stream work still uses them; they carry
// the second stream's mark, which their first use on the context stream waits for, and what
// the program reads stays referenced until then.  False when this does not apply (nothing
// launched): the chain then runs on the context stream.
bool side_flush(Backend* be, const Walk& w, const Program& prog, const std::vector<int>& out_idx) {
  if (!be->opt.overlap || be->on_side || be->recent.empty() || w.leaves.empty()) return false;
  const size_t n = w.order.back()->n;
  if (n == 0) return false;
  std::vector<Node*> src(w.leaves.size());  // the nodes read (a broadcast reads its source)
  uint64_t need = 0;
  for (size_t i = 0; i < w.leaves.size(); ++i) {
    Node* lf = w.leaves[i];
    Node* x = lf->kind == Kind::kBcast ? lf->lhs : lf;
    // computed, contiguous, its own memory (not an arena slice), never updated in place
    if (!x || x->kind != Kind::kValue || !x->buf || x->buf->owner || !x->tshape.empty() || x->in_place) return false;
    src[i] = x;
    if (!x->side_made) need = std::max(need, x->done_seq + 1);
  }
  // The earliest mark after the inputs for which cached blocks released before it can take
  // the outputs; not the latest mark, so that a product launched after it runs beside.
  MarkP wait;
  for (size_t i = 0; i + 1 < be->recent.size(); ++i) {
    const MarkP& m = be->recent[i];
    if (m->seq >= need && ctx_count_released_by(be->ctx, 4 * n, m->clock) >= out_idx.size()) {
      wait = m;
      break;
    }
  }
  if (!wait) return false;
  std::vector<BufP> bufs;
  for (size_t i = 0; i < out_idx.size(); ++i) {
    void* p = ctx_allocate_released_by(be->ctx, 4 * n, wait->clock);
    if (!p) fail(ORCA_HIP_ERR_INTERNAL, "side_flush: a counted cached block was not there");
    bufs.push_back(own(be->ctx, p, 4 * n));
  }
  std::vector<orca_hip_ew_input> ins(w.leaves.size());
  for (size_t i = 0; i < w.leaves.size(); ++i) {
    Node* lf = w.leaves[i];
    ins[i].ptr = src[i]->buf->ptr;
    ins[i].div = lf->kind == Kind::kBcast ? lf->div : 1;
    ins[i].mod = lf->kind == Kind::kBcast ? lf->mod : n;
  }
  std::vector<float*> outs;
  for (auto& b : bufs) outs.push_back(b->ptr);
  // As the fused optimizer pass splits its second-stream part: side_frac of the elements on
  // side_bpc blocks per CU beside the product after `wait`, the rest on the full grid after
  // the mark before the latest (beside the last product, which leaves CUs idle).  Only a
  // program without broadcast inputs splits (its element ranges are independent).
  MarkP mid;
  for (auto& m : be->recent)
    if (m->seq > wait->seq && m != be->recent.back()) mid = m;
  bool plain = true;
  for (Node* lf : w.leaves) plain = plain && lf->kind != Kind::kBcast;
  size_t n1 = n;
  if (mid && plain && be->opt.side_frac < 1.0) {
    n1 = (size_t)((double)n * std::max(0.0, be->opt.side_frac)) / 64 * 64;  // 256-byte aligned split
    if (n1 == 0) n1 = n;
  }
  struct Part {
    size_t from, cnt;
    MarkP after;
    int bpc;
  };
  const int bpc = be->opt.side_bpc > 0 ? be->opt.side_bpc : -1;
  std::vector<Part> parts;
  if (n1 < n) {
    parts.push_back(Part{0, n1, wait, bpc});
    parts.push_back(Part{n1, n - n1, mid, -1});
  } else {
    parts.push_back(Part{0, n, wait, bpc});
  }
  int rc = ORCA_HIP_OK;
  MarkP done;
  for (size_t i = 0; i < parts.size() && rc == ORCA_HIP_OK; ++i) {
    const Part& pt = parts[i];
    rc = orca_hip_use_side_stream(be->ctx, pt.bpc);
    if (rc != ORCA_HIP_OK) break;
    be->on_side = true;
    std::vector<orca_hip_ew_input> in = ins;
    std::vector<float*> o = outs;
    if (pt.cnt != n) {  // a range of the elements (every input is read elementwise)
      for (auto& x : in) {
        x.ptr += pt.from;
        x.mod = pt.cnt;
      }
      for (auto& q : o) q += pt.from;
    }
    rc = orca_hip_event_wait(be->ctx, pt.after->ev);
    if (rc == ORCA_HIP_OK)
      rc = orca_hip_ew_program(be->ctx, pt.cnt, in.data(), in.size(), o.data(), prog.oregs.data(), o.size(),
                               prog.instrs.data(), prog.instrs.size(), prog.n_regs);
    if (rc == ORCA_HIP_OK && i + 1 == parts.size()) rc = guard_nodes([&] { done = new_mark(be); });
    be->on_side = false;
    const int rc2 = orca_hip_use_side_stream(be->ctx, 0);
    if (rc == ORCA_HIP_OK) rc = rc2;
  }
  ck(rc);
  for (Node* x : src) done->keep.push_back(ref(x));
  for (size_t i = 0; i < out_idx.size(); ++i) {
    Node* o = w.order[out_idx[i]];
    set_value(o, bufs[i]);
    o->side_made = true;
    o->ready = done;
  }
  return true;
}

// Runs root's pending chain as one program.  Pending values in the chain referenced from
// outside it (beyond the chain's own operand links) are written too.  A chain's program is
// compiled once per structure -- opcodes, operand slots, outputs -- and reused with the
// chain's scalars written into it.  Falls back to running the operands' chains first when
// the program would exceed the interpreter's registers or outputs.
void flush(Backend* be, Node* root) {
  if (root->kind != Kind::kEw) return;
  Walk w;
  w.visit(root);
  std::vector<int> out_idx;
  const int n_ops = (int)w.order.size();
  for (int k = 0; k + 1 < n_ops; ++k) {
    Node* x = w.order[k];
    if (x->rc.load(std::memory_order_relaxed) > w.inner[x]) out_idx.push_back(k);
  }
  out_idx.push_back(n_ops - 1);  // the root
  // a product first input held beyond the chain's one link to it
  const bool prod_shared = w.leaves[0]->rc.load(std::memory_order_relaxed) > 1;
  // hold the chain while inputs are computed (which may run other chains)
  std::vector<Ref> hold;
  hold.reserve(w.order.size() + w.leaves.size());
  for (Node* x : w.order) hold.emplace_back(ref(x));
  for (Node* x : w.leaves) hold.emplace_back(ref(x));
  if (be->opt.fold && w.leaves[0]->kind == Kind::kProd && fold_chain(be, w, out_idx, prod_shared)) return;
  std::string key(reinterpret_cast<const char*>(w.sig.data()), w.sig.size() * sizeof(int));
  key.append("|");
  key.append(reinterpret_cast<const char*>(out_idx.data()), out_idx.size() * sizeof(int));
  key.append(std::to_string(w.leaves.size()));
  auto it = be->programs.find(key);
  if (it == be->programs.end()) it = be->programs.emplace(key, compile(w, out_idx)).first;
  Program& prog = it->second;
  if (!prog.ok) {
    hold.clear();
    flush_operands_first(be, root);
    return;
  }
  for (int k : prog.scalar_at) prog.instrs[k].scalar = w.scalars[k];
  if (side_flush(be, w, prog, out_idx)) return;
  const size_t n = root->n;
  std::vector<orca_hip_ew_input> ins(std::max<size_t>(1, w.leaves.size()));
  for (size_t i = 0; i < w.leaves.size(); ++i) {
    Node* lf = w.leaves[i];
    if (lf->kind == Kind::kBcast) {
      ins[i].ptr = dptr(be, lf->lhs);
      ins[i].div = lf->div;
      ins[i].mod = lf->mod;
    } else {
      ins[i].ptr = dptr(be, lf);
      ins[i].div = 1;
      ins[i].mod = n;
    }
  }
  std::vector<BufP> bufs;
  std::vector<float*> outs;
  for (size_t i = 0; i < out_idx.size(); ++i) {
    bufs.push_back(alloc_buf(be, n));
    outs.push_back(bufs.back()->ptr);
  }
  ck(orca_hip_ew_program(be->ctx, n, ins.data(), w.leaves.size(), outs.data(), prog.oregs.data(), outs.size(),
                         prog.instrs.data(), prog.instrs.size(), prog.n_regs));
  for (size_t i = 0; i < out_idx.size(); ++i) set_value(w.order[out_idx[i]], bufs[i]);
}

// Runs root's pending chain as flush does, together with the row reduction
// sum_to_shape / max_to_shape([rows, cols] -> [rows, 1]) of its value, in one launch
// (orca_hip_ew_program_rows, whose rows have the bits of the one-by-one reduction).  Null,
// with nothing run, when the chain does not qualify: a chain headed by a pending product
// (left to the product's epilogue), rows wider than the launch takes, a program past the
// interpreter's limits, or launches going to the second stream.
Node* chain_rows(Backend* be, Node* root, size_t rows, size_t cols, bool is_max) {
  if (root->kind != Kind::kEw || be->on_side || cols == 0 || cols > 64 || rows * cols != root->n ||
      rows > ((size_t)1 << 31) / cols)
    return nullptr;
  Walk w;
  w.visit(root);
  if (be->opt.fold && w.leaves[0]->kind == Kind::kProd) return nullptr;
  std::vector<int> out_idx;
  const int n_ops = (int)w.order.size();
  for (int k = 0; k + 1 < n_ops; ++k) {
    Node* x = w.order[k];
    if (x->rc.load(std::memory_order_relaxed) > w.inner[x]) out_idx.push_back(k);
  }
  out_idx.push_back(n_ops - 1);  // the root
  std::string key(reinterpret_cast<const char*>(w.sig.data()), w.sig.size() * sizeof(int));
  key.append("|");
  key.append(reinterpret_cast<const char*>(out_idx.data()), out_idx.size() * sizeof(int));
  key.append(std::to_string(w.leaves.size()));
  auto it = be->programs.find(key);
  if (it == be->programs.end()) it = be->programs.emplace(key, compile(w, out_idx)).first;
  Program& prog = it->second;
  if (!prog.ok) return nullptr;
  std::vector<Ref> hold;
  hold.reserve(w.order.size() + w.leaves.size());
  for (Node* x : w.order) hold.emplace_back(ref(x));
  for (Node* x : w.leaves) hold.emplace_back(ref(x));
  for (int k : prog.scalar_at) prog.instrs[k].scalar = w.scalars[k];
  const size_t n = root->n;
  std::vector<orca_hip_ew_input> ins(std::max<size_t>(1, w.leaves.size()));
  for (size_t i = 0; i < w.leaves.size(); ++i) {
    Node* lf = w.leaves[i];
    if (lf->kind == Kind::kBcast) {
      ins[i].ptr = dptr(be, lf->lhs);
      ins[i].div = lf->div;
      ins[i].mod = lf->mod;
    } else {
      ins[i].ptr = dptr(be, lf);
      ins[i].div = 1;
      ins[i].mod = n;
    }
  }
  std::vector<BufP> bufs;
  std::vector<float*> outs;
  for (size_t i = 0; i < out_idx.size(); ++i) {
    bufs.push_back(alloc_buf(be, n));
    outs.push_back(bufs.back()->ptr);
  }
  BufP red = alloc_buf(be, rows);
  ck(orca_hip_ew_program_rows(be->ctx, rows, cols, ins.data(), w.leaves.size(), outs.data(), prog.oregs.data(),
                              outs.size(), prog.instrs.data(), prog.instrs.size(), prog.n_regs, prog.oregs.back(),
                              is_max ? 1 : 0, red->ptr));
  for (size_t i = 0; i < out_idx.size(); ++i) set_value(w.order[out_idx[i]], bufs[i]);
  return value_node(be, rows, std::move(red));
}

// ---- creating pending nodes
bool is_lazy_f32(Backend* be, int dtype) { return be->opt.lazy && dtype == ORCA_HIP_F32; }

// The reference's optimizers update the parameters one after another, so the update that
// reads one weight or bias gradient is complete once the update after it has started.  When
// an op reads a gradient g (the previous one read being `prev`), every pending chain that
// reads a gradient other than those two and whose inputs are all computed runs now rather
// than at its first use: while the backward's last products may still run, so that the ones
// on the second stream run beside them.  (Not at the first read after it: the finished
// update's temporaries can still be held by the caller then, and would be written out.)
void flush_finished_updates(Backend* be, const Node* g, const Node* prev) {
  std::unordered_set<const Node*> consumed;  // operands of pending nodes
  for (auto& kv : be->pending) {
    const Node* p = kv.second;
    for (int i = 0; i < p->nopd; ++i) consumed.insert(p->opd[i]);
    if (p->lhs) consumed.insert(p->lhs);
    if (p->rhs) consumed.insert(p->rhs);
  }
  std::vector<Ref> roots;
  for (auto& kv : be->pending) {
    Node* p = kv.second;
    if (p->kind != Kind::kEw || consumed.count(p)) continue;
    Walk w;
    w.visit(p);
    bool ready = true, other_grad = false;
    for (Node* lf : w.leaves) {
      Node* x = lf->kind == Kind::kBcast ? lf->lhs : lf;
      if (!x || x->kind != Kind::kValue) {
        ready = false;
        break;
      }
      if (x->made && x != g && x != prev) other_grad = true;
    }
    if (ready && other_grad) roots.emplace_back(ref(p));
  }
  for (auto& r : roots)
    if (r->kind == Kind::kEw) flush(be, r.get());
}

// A pending elementwise op over equally long operands (transposed views are
// materialised first).  Operands whose pending chains would push this one past the
// interpreter's limits are run first.
Node* ew(Backend* be, uint8_t op, std::vector<Ref> opds, size_t n, float scalar = 0.0f) {
  for (auto& o : opds)
    if (o->kind != Kind::kBcast && !o->tshape.empty()) o = plain(be, o.get());
  if (be->opt.overlap && be->opt.lazy && !be->on_side) {
    for (auto& o : opds) {
      if (o->kind != Kind::kBcast && o->made && o.get() != be->grad_read) {
        const Node* prev = be->grad_read;
        be->grad_read = o.get();  // compared by address only
        flush_finished_updates(be, o.get(), prev);
        break;
      }
    }
  }
  int ops, leaves;
  for (;;) {
    ops = 1;
    leaves = 0;
    for (auto& o : opds) {
      if (o->kind == Kind::kEw) {
        ops += o->ew_ops;
        leaves += o->ew_leaves;
      } else {
        leaves += 1;
      }
    }
    if (ops <= ORCA_HIP_EW_MAX_OPS / 2 && leaves <= ORCA_HIP_EW_MAX_INPUTS) break;
    Node* biggest = nullptr;
    for (auto& o : opds)
      if (o->kind == Kind::kEw && (!biggest || o->ew_ops > biggest->ew_ops)) biggest = o.get();
    flush(be, biggest);
  }
  Node* x = new_node(be, n);
  x->kind = Kind::kEw;
  x->op = op;
  x->nopd = (uint8_t)opds.size();
  for (size_t i = 0; i < opds.size(); ++i) x->opd[i] = opds[i].release();
  x->scalar = scalar;
  x->ew_ops = ops;
  x->ew_leaves = leaves;
  track_pending(be, x);
  return x;
}

Node* bcast(Backend* be, Node* src, size_t n, uint64_t div, uint64_t mod) {
  Node* b = new_node(be, n);
  b->kind = Kind::kBcast;
  b->lhs = ref(src);
  b->div = div;
  b->mod = mod;
  return b;
}

bool same_len(std::initializer_list<Node*> xs) {
  const size_t n = (*xs.begin())->n;
  for (Node* x : xs)
    if (x->n != n) return false;
  return true;
}

// A one-element upload kept on the host until the device needs it; n > 1 gives its
// single-value broadcast to n elements.
Node* const_node(Backend* be, float value, size_t n) {
  Node* c = new_node(be, 1);
  c->kind = Kind::kConst;
  c->has_const = true;
  c->cval = value;
  if (n == 1) return c;
  Ref cr(c);
  std::vector<Ref> o;
  o.emplace_back(bcast(be, c, n, 1, 1));
  return ew(be, ORCA_HIP_EW_COPY, std::move(o), n);
}

// The one-element constant whose value s holds everywhere, or null.
Node* const_src(Node* s) {
  if (s->has_const) return s;
  if (s->kind == Kind::kEw && s->op == ORCA_HIP_EW_COPY) {
    Node* b = s->opd[0];
    if (b->kind == Kind::kBcast && b->mod == 1 && b->lhs->has_const) return b->lhs;
  }
  return nullptr;
}

// add / mul with a constant operand as a scalar instruction (x + c, x * c: the ops' own f32
// operations; the constant is never NaN, so the operand order does not matter), or of two
// constants on the host; null when neither operand is a constant.
Node* fold_const(Backend* be, uint8_t op, Node* a, Node* b) {
  Node* ca = const_src(a);
  Node* cb = const_src(b);
  if (!ca && !cb) return nullptr;
  const size_t n = a->n;
  if (ca && cb) {
    volatile float x = ca->cval, y = cb->cval;
    const float v = op == ORCA_HIP_EW_ADD ? x + y : x * y;
    if (std::isnan(v)) return nullptr;
    return const_node(be, v, n);
  }
  Node* x = cb ? a : b;
  const float c = cb ? cb->cval : ca->cval;
  // x * 1 is x bit for bit unless x is a signaling NaN (the multiply would quiet it), which
  // arithmetic never leaves (denormals are kept, as the op's own kernel keeps them)
  if (op == ORCA_HIP_EW_MUL && c == 1.0f && x->kind == Kind::kValue && x->quiet && x->tshape.empty()) return ref(x);
  std::vector<Ref> o;
  o.emplace_back(ref(x));
  return ew(be, op == ORCA_HIP_EW_ADD ? ORCA_HIP_EW_ADD_SCALAR : ORCA_HIP_EW_MUL_SCALAR, std::move(o), n, c);
}

// Before an in-place update: values derived lazily from these storages are computed
// from their current contents, and their memoised identity reductions are dropped.
template <class Targets>
void mutating(Backend* be, const Targets& targets) {
  flush_all(be);
  for (Node* s : targets) {
    if (!s) continue;
    s->in_place = true;
    std::vector<Node*> ws = s->waiters;
    for (Node* t : ws) {
      Ref tt(ref(t));
      materialize(be, t);
    }
    for (Node* t : s->waiters) t->lhs = nullptr;  // defensive: a run waiter leaves the list
    s->waiters.clear();
    if (s->ident) {
      s->ident->ident_of = nullptr;
      s->ident = nullptr;
    }
    if (s->has_const) {
      materialize(be, s);  // a constant not yet on the device is uploaded before it changes there
      s->has_const = false;
    }
  }
}

// (div, mod) when expanding in_shape to out_shape reads input element (e / div) % mod for
// output element e (the input's non-broadcast dims are one contiguous block of the output's).
bool broadcast_map(const size_t* in_shape, size_t in_rank, const size_t* out_shape, size_t out_rank, uint64_t* div,
                   uint64_t* mod) {
  if (out_rank < in_rank) return false;
  std::vector<size_t> pin(out_rank, 1);
  for (size_t i = 0; i < in_rank; ++i) pin[out_rank - in_rank + i] = in_shape[i];
  std::vector<size_t> kept;
  for (size_t d = 0; d < out_rank; ++d)
    if (pin[d] != 1) kept.push_back(d);
  for (size_t d : kept)
    if (pin[d] != out_shape[d]) return false;
  if (kept.empty()) {
    *div = 1;
    *mod = 1;
    return true;
  }
  const size_t i0 = kept.front(), i1 = kept.back() + 1;
  for (size_t d = i0; d < i1; ++d)
    if (pin[d] == 1 && out_shape[d] != 1) return false;
  uint64_t dv = 1, md = 1;
  for (size_t d = i1; d < out_rank; ++d) dv *= out_shape[d];
  for (size_t d = i0; d < i1; ++d) md *= out_shape[d];
  *div = dv;
  *mod = md;
  return true;
}

// ---- the optimizer pass (rows of p_src, p_dst, g, m, v, n)
struct Row {
  Node* p_src;
  Node* p_dst;
  Node* g;
  Node* m;
  Node* v;
  size_t n;
};

struct PtrRow {
  float* p_src;
  float* p_dst;
  const float* g;
  float* m;
  float* v;
  size_t n;
};

// Splits rows at `frac` of their elements, on a 64-element boundary (256 bytes, so a split
// segment keeps its alignment).
void split_rows(const std::vector<PtrRow>& rows, double frac, std::vector<PtrRow>& a, std::vector<PtrRow>& b) {
  size_t total = 0;
  for (auto& r : rows) total += r.n;
  const size_t cut = (size_t)((double)total * frac) / 64 * 64;
  size_t acc = 0;
  for (auto& r : rows) {
    if (acc + r.n <= cut) {
      a.push_back(r);
    } else if (acc >= cut) {
      b.push_back(r);
    } else {
      const size_t k = (cut - acc) / 64 * 64;
      PtrRow x = r, y = r;
      x.n = k;
      auto sh = [k](auto* p) { return p ? p + k : p; };
      y.p_src = sh(r.p_src);
      y.p_dst = sh(r.p_dst);
      y.g = sh(r.g);
      y.m = sh(r.m);
      y.v = sh(r.v);
      y.n = r.n - k;
      if (x.n) a.push_back(x);
      if (y.n) b.push_back(y);
    }
    acc += r.n;
  }
}

template <class Launch>
void optimizer_pass(Backend* be, std::vector<Row>& rows, bool has_moments, Launch launch) {
  // launch(vector<PtrRow>) runs the pass over those rows on the current stream.
  be->marking = be->opt.overlap != 0;
  if (be->opt.overlap)  // gradients still pending run now, the last parameter's last (backward order)
    for (auto it = rows.rbegin(); it != rows.rend(); ++it)
      if (it->g->pending()) materialize(be, it->g);
  std::vector<MarkP> marks;
  uint64_t last = 0;
  bool any = false;
  if (be->opt.overlap) {
    for (auto& r : rows) {
      marks.push_back(r.g->made);
      if (r.g->made) {
        last = any ? std::max(last, r.g->made->seq) : r.g->made->seq;
        any = true;
      }
    }
  }
  std::vector<size_t> side, here;
  MarkP after;
  for (size_t i = 0; i < rows.size(); ++i) {
    const MarkP& m = be->opt.overlap ? marks[i] : MarkP();
    if (m && m->seq != last) {
      side.push_back(i);
      if (!after || m->seq > after->seq) after = m;  // the same stream's earlier marks come before it
    } else {
      here.push_back(i);
    }
  }
  auto ptrs_of = [&](const Row& r) {
    PtrRow p;
    p.p_src = dptr(be, r.p_src);
    p.p_dst = dptr(be, r.p_dst);
    p.g = dptr(be, r.g);
    p.m = has_moments ? dptr(be, r.m) : nullptr;
    p.v = has_moments ? dptr(be, r.v) : nullptr;
    p.n = r.n;
    return p;
  };
  if (!side.empty()) {
    MarkP mid;
    for (auto& m : be->recent)
      if (m->seq > after->seq && m->seq < last && (!mid || m->seq > mid->seq)) mid = m;
    std::vector<PtrRow> ptrs;  // pending values settled on the context stream first
    for (size_t i : side) ptrs.push_back(ptrs_of(rows[i]));
    struct Part {
      MarkP mark;
      int bpc;
      std::vector<PtrRow> rows;
    };
    std::vector<Part> parts;
    const int bpc = be->opt.side_bpc > 0 ? be->opt.side_bpc : -1;
    if (mid && be->opt.side_frac < 1.0) {
      Part a{after, bpc, {}}, b{mid, -1, {}};
      split_rows(ptrs, be->opt.side_frac, a.rows, b.rows);
      parts.push_back(std::move(a));
      parts.push_back(std::move(b));
    } else {
      parts.push_back(Part{after, bpc, ptrs});
    }
    MarkP done;
    for (auto& part : parts) {
      if (part.rows.empty()) continue;
      ck(orca_hip_use_side_stream(be->ctx, part.bpc));
      be->on_side = true;
      int rc = orca_hip_event_wait(be->ctx, part.mark->ev);
      if (rc == ORCA_HIP_OK) rc = guard_nodes([&] { launch(part.rows); });
      MarkP d;
      if (rc == ORCA_HIP_OK) rc = guard_nodes([&] { d = new_mark(be); });  // the side stream's work so far
      be->on_side = false;
      const int rc2 = orca_hip_use_side_stream(be->ctx, 0);
      ck(rc);
      ck(rc2);
      done = d;
    }
    if (done) {
      for (size_t i : side) {  // what the side pass only reads stays referenced until the wait
        done->keep.push_back(ref(rows[i].p_src));
        done->keep.push_back(ref(rows[i].g));
      }
      for (size_t i : side) {
        rows[i].p_dst->ready = done;
        if (has_moments) {
          rows[i].m->ready = done;
          rows[i].v->ready = done;
        }
      }
    }
  }
  if (!here.empty()) {
    std::vector<PtrRow> ptrs;
    for (size_t i : here) ptrs.push_back(ptrs_of(rows[i]));
    launch(ptrs);
  }
}

std::vector<orca_hip_opt_segment> segments(const std::vector<PtrRow>& rows, size_t from, size_t count) {
  std::vector<orca_hip_opt_segment> segs;
  for (size_t i = from; i < from + count; ++i) {
    orca_hip_opt_segment s{};
    s.p_src = rows[i].p_src;
    s.p_dst = rows[i].p_dst;
    s.g = rows[i].g;
    s.m = rows[i].m;
    s.v = rows[i].v;
    s.n = rows[i].n;
    segs.push_back(s);
  }
  return segs;
}

// ---- argument checks
Node* arg(Backend* be, orca_hip_storage* s, const char* what) {
  if (!s) fail(ORCA_HIP_ERR_INTERNAL, std::string("null storage (") + what + ")");
  Node* x = N_(s);
  if (x->be != be) {
    int d0 = 0, d1 = 0;
    (void)orca_hip_device(be->ctx, &d0);
    (void)orca_hip_device(x->be->ctx, &d1);
    if (d0 != d1) fail_device(d0, d1);
    fail(ORCA_HIP_ERR_INTERNAL, "storage belongs to another context on the same device");
  }
  return x;
}

void check_out(void* out) {
  if (!out) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
}

std::string shape_string(const size_t* shape, size_t rank) {
  std::string s = "[";
  for (size_t i = 0; i < rank; ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
  return s + "]";
}

// Entry-point scaffolding: lock, run, return a node through `out`.
template <class F>
int entry(orca_hip_backend* h, F&& f) {
  return guard_nodes([&] {
    if (!h) fail(ORCA_HIP_ERR_INTERNAL, "null orca_hip_backend");
    Planner* pl = h->pl;
    std::lock_guard<std::mutex> lk(pl->mu);
    pl->opt = h->opt;
    f(pl);
  });
}

void put(orca_hip_storage** out, Node* x) { *out = S_(x); }

// A kernel entry point of the buffer-level ABI that returns a new buffer of n floats.
template <class Call>
Node* kernel_node(Backend* be, size_t n, Call call) {
  void* out = nullptr;
  ck(call(&out));
  return value_node(be, n, own(be->ctx, out, 4 * std::max<size_t>(n, 1)));
}

typedef int (*Ew1Fn)(orca_hip_ctx*, const void*, const size_t*, size_t, int, void**);
typedef int (*Ew2Fn)(orca_hip_ctx*, const void*, const void*, const size_t*, size_t, int, void**);

Node* unary(Backend* be, uint8_t op, Ew1Fn fn, Node* s, const size_t* shape, size_t rank, int dtype) {
  if (is_lazy_f32(be, dtype)) {
    std::vector<Ref> o;
    o.emplace_back(ref(s));
    return ew(be, op, std::move(o), s->n);
  }
  Ref p = plain(be, s);
  float* sp = dptr(be, p.get());
  return kernel_node(be, numel_of(shape, rank), [&](void** out) { return fn(be->ctx, sp, shape, rank, dtype, out); });
}

Node* binary(Backend* be, uint8_t op, Ew2Fn fn, Node* a, Node* b, const size_t* shape, size_t rank, int dtype) {
  if (is_lazy_f32(be, dtype) && same_len({a, b})) {
    std::vector<Ref> o;
    o.emplace_back(ref(a));
    o.emplace_back(ref(b));
    return ew(be, op, std::move(o), a->n);
  }
  Ref pa = plain(be, a), pb = plain(be, b);
  float* ap = dptr(be, pa.get());
  float* bp = dptr(be, pb.get());
  return kernel_node(be, numel_of(shape, rank),
                     [&](void** out) { return fn(be->ctx, ap, bp, shape, rank, dtype, out); });
}

typedef int (*ReshapeFn)(orca_hip_ctx*, const void*, const size_t*, size_t, const size_t*, size_t, int, void**);

Node* reshape_like(Backend* be, ReshapeFn fn, Node* s, const size_t* in_shape, size_t in_rank, const size_t* out_shape,
                   size_t out_rank, int dtype) {
  Ref p = plain(be, s);
  float* sp = dptr(be, p.get());
  return kernel_node(be, numel_of(out_shape, out_rank),
                     [&](void** out) { return fn(be->ctx, sp, in_shape, in_rank, out_shape, out_rank, dtype, out); });
}

// A pending column sum sum_to_shape(s, [rows, cols] -> [1, cols]).
Node* deferred_colsum(Backend* be, Node* s, size_t rows, size_t cols) {
  Node* x = new_node(be, cols);
  x->kind = Kind::kColsum;
  x->lhs = ref(s);
  x->M = rows;
  x->N = cols;
  s->waiters.push_back(x);
  return x;
}

// Whether a pending product G W^T ([rows, k] x [k, cols] with W^T a view) waits beside a
// weight gradient of G.
bool pending_input_gradient(Backend* be, Node* g, size_t rows, size_t k, size_t cols) {
  for (auto& kv : be->pending) {
    const Node* p = kv.second;
    if (p->kind == Kind::kProd && p->lhs == g && p->rt && !p->lt && p->M == rows && p->K == k && p->N == cols)
      return true;
  }
  return false;
}

// Removes and returns a still-pending column sum of s with `cols` columns (null if none).
Node* take_colsum_waiter(Node* s, size_t cols) {
  for (size_t i = 0; i < s->waiters.size(); ++i) {
    Node* t = s->waiters[i];
    if (t->kind == Kind::kColsum && t->n == cols) return t;
  }
  return nullptr;
}

[[noreturn]] void unsupported(const char* op, int dtype) { fail_dtype(op, dtype); }

}  // namespace
}  // namespace orca_hip

using namespace orca_hip;

// ============================================================== C ABI
extern "C" {

int orca_hip_last_error_info(orca_hip_error_info* out) {
  if (!out) return ORCA_HIP_ERR_INTERNAL;
  last_error_info(out);
  return ORCA_HIP_OK;
}

int orca_hip_backend_default_options(orca_hip_backend_options* out) {
  return guard_nodes([&] {
    check_out(out);
    out->lazy = 1;
    out->deferred = 1;
    out->fold = 1;
    out->overlap = 1;
    out->side_frac = 0.7;
    out->side_bpc = 3;
    if (const char* v = std::getenv("ORCA_HIP_OVERLAP")) out->overlap = v[0] != '0';
    if (const char* v = std::getenv("ORCA_HIP_OPT_SIDE_FRAC")) out->side_frac = std::atof(v) / 100.0;
    if (const char* v = std::getenv("ORCA_HIP_OPT_SIDE_BPC")) out->side_bpc = std::atoi(v) ? std::atoi(v) : -1;
  });
}

int orca_hip_backend_create(orca_hip_ctx* ctx, const orca_hip_backend_options* opts, orca_hip_backend** out) {
  return guard_nodes([&] {
    check_ctx(ctx);
    check_out(out);
    orca_hip_backend_options o{};
    if (opts) {
      o = *opts;
    } else {
      ck(orca_hip_backend_default_options(&o));
    }
    if (!o.lazy) o.fold = 0;  // folds need pending products
    auto* h = new orca_hip_backend();
    h->opt = o;
    h->pl = planner_for(ctx);
    *out = h;
  });
}

int orca_hip_backend_destroy(orca_hip_backend* be) {
  return guard_nodes([&] {
    if (!be) return;
    Planner* pl = be->pl;
    delete be;
    if (pl->rc.load() == 1) {  // the last handle, and no storage left
      std::lock_guard<std::mutex> lk(pl->mu);
      pl->recent.clear();  // their events go back to the context
      pl->programs.clear();
    }
    backend_unref(pl);
  });
}

int orca_hip_storage_retain(orca_hip_storage* s) {
  if (!s) return ORCA_HIP_ERR_INTERNAL;
  ref(N_(s));
  return ORCA_HIP_OK;
}

int orca_hip_storage_release(orca_hip_storage* s) {
  return guard_nodes([&] {
    if (!s) return;
    Node* x = N_(s);
    Backend* be = x->be;
    be->rc.fetch_add(1, std::memory_order_relaxed);  // the backend outlives the lock below
    {
      std::lock_guard<std::mutex> lk(be->mu);
      unref(x);
    }
    backend_unref(be);
  });
}

int orca_hip_storage_len(const orca_hip_storage* s, size_t* n) {
  if (!s || !n) return ORCA_HIP_ERR_INTERNAL;
  *n = reinterpret_cast<const Node*>(s)->n;
  return ORCA_HIP_OK;
}

int orca_hip_storage_flags(const orca_hip_storage* s, uint32_t* flags) {
  if (!s || !flags) return ORCA_HIP_ERR_INTERNAL;
  const Node* x = reinterpret_cast<const Node*>(s);
  std::lock_guard<std::mutex> lk(x->be->mu);
  uint32_t f = 0;
  if (x->pending()) f |= ORCA_HIP_STORAGE_PENDING;
  if (!x->tshape.empty()) f |= ORCA_HIP_STORAGE_TRANSPOSED;
  if (x->ready) f |= ORCA_HIP_STORAGE_MARKED;
  if (x->has_const) f |= ORCA_HIP_STORAGE_CONSTANT;
  *flags = f;
  return ORCA_HIP_OK;
}

int orca_hip_storage_device_ptr(orca_hip_backend* be, orca_hip_storage* s, void** ptr) {
  return entry(be, [&](Backend* b) {
    check_out(ptr);
    *ptr = dptr(b, arg(b, s, "device_ptr"));
  });
}

// ---------------------------------------------------------------- trait methods
int orca_hip_trait_device(orca_hip_backend* be, int* kind, int* index) {
  return entry(be, [&](Backend* b) {
    if (!kind || !index) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    int d = 0;
    ck(orca_hip_device(b->ctx, &d));
    *kind = 2;  // Device::Gpu
    *index = d;
  });
}

int orca_hip_trait_zeros(orca_hip_backend* be, const size_t* shape, size_t rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    put(out, kernel_node(b, numel_of(shape, rank), [&](void** o) { return orca_hip_zeros(b->ctx, shape, rank, dtype, o); }));
  });
}

int orca_hip_trait_from_f32_slice(orca_hip_backend* be, const size_t* shape, size_t rank, const float* data, size_t n,
                                  orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    if (b->opt.lazy && n == 1 && numel_of(shape, rank) == 1 && data && !std::isnan(data[0])) {
      put(out, const_node(b, data[0], 1));
      return;
    }
    put(out, kernel_node(b, n, [&](void** o) { return orca_hip_from_f32_slice(b->ctx, shape, rank, data, n, o); }));
  });
}

int orca_hip_trait_to_f32_vec(orca_hip_backend* be, orca_hip_storage* s, float* host, size_t n) {
  return entry(be, [&](Backend* b) {
    Ref p = plain(b, arg(b, s, "to_f32_vec"));
    if (n != p->n)
      fail_shape("to_f32_vec", std::to_string(p->n) + " elements", std::to_string(n) + " elements");
    ck(orca_hip_to_f32_vec(b->ctx, dptr(b, p.get()), n, host));
  });
}

int orca_hip_trait_matmul(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* lhs_shape,
                          size_t lhs_rank, const size_t* rhs_shape, size_t rhs_rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* l = arg(b, lhs, "matmul lhs");
    Node* r = arg(b, rhs, "matmul rhs");
    const bool two_d = dtype == ORCA_HIP_F32 && lhs_rank == 2 && rhs_rank == 2 && lhs_shape[1] == rhs_shape[0];
    // the weight gradient X^T G of a storage whose bias column sum is pending: both in one launch
    if (two_d && b->opt.deferred && !r->waiters.empty() && r->tshape.empty()) {
      const size_t M = lhs_shape[0], K = lhs_shape[1], N = rhs_shape[1];
      Node* target = take_colsum_waiter(r, N);
      if (target) {
        Ref t(ref(target));
        const int lv = l->tshape.empty() ? ORCA_HIP_VIEW_CONTIGUOUS : ORCA_HIP_VIEW_TRANSPOSED;
        // A classifier head's weight gradient (G with at most 16 columns) waits for the input
        // gradient G W^T pending beside it: both, and this bias gradient, then run from one grid.
        if (b->opt.fold && lv == ORCA_HIP_VIEW_TRANSPOSED && N <= 16 && M > 0 && K > 0 &&
            pending_input_gradient(b, r, K, N, M)) {
          Node* x = new_node(b, M * N);
          x->kind = Kind::kProd;
          x->lhs = ref(l);
          x->rhs = ref(r);
          x->M = M;
          x->K = K;
          x->N = N;
          x->lt = true;
          x->cs = ref(target);
          target->via = x;
          track_pending(b, x);
          put(out, x);
          return;
        }
        float* lp = dptr(b, l);
        float* rp = dptr(b, r);
        BufP cs = alloc_buf(b, N);
        void* o = nullptr;
        const bool mark = marking(b);
        orca_hip_event* ev = nullptr;
        ck(orca_hip_matmul_ev(b->ctx, lp, rp, M, K, N, lv, ORCA_HIP_VIEW_CONTIGUOUS, dtype, cs->ptr, &o,
                              mark ? &ev : nullptr));
        set_value(target, cs);
        Node* res = value_node(b, M * N, own(b->ctx, o, 4 * M * N));
        if (mark) {
          MarkP m = record_mark(b, ev);
          if (lv == ORCA_HIP_VIEW_TRANSPOSED) res->made = target->made = m;  // a weight gradient and its bias gradient
        }
        put(out, res);
        return;
      }
    }
    if (two_d && b->opt.lazy) {
      const size_t M = lhs_shape[0], K = lhs_shape[1], N = rhs_shape[1];
      if (l->n == M * K && r->n == K * N && M * N > 0 && K > 0) {
        Node* x = new_node(b, M * N);
        x->kind = Kind::kProd;
        x->lhs = ref(l);
        x->rhs = ref(r);
        x->M = M;
        x->K = K;
        x->N = N;
        x->lt = !l->tshape.empty();
        x->rt = !r->tshape.empty();
        track_pending(b, x);
        put(out, x);
        return;
      }
    }
    size_t n = 1;
    for (size_t i = 0; i + 1 < lhs_rank; ++i) n *= lhs_shape[i];
    n *= rhs_rank ? rhs_shape[rhs_rank - 1] : 1;
    const int lv = l->tshape.empty() ? ORCA_HIP_VIEW_CONTIGUOUS : ORCA_HIP_VIEW_TRANSPOSED;
    const int rv = r->tshape.empty() ? ORCA_HIP_VIEW_CONTIGUOUS : ORCA_HIP_VIEW_TRANSPOSED;
    float* lp = dptr(b, l);
    float* rp = dptr(b, r);
    put(out, kernel_node(b, n, [&](void** o) {
          return orca_hip_matmul(b->ctx, lp, rp, lhs_shape, lhs_rank, rhs_shape, rhs_rank, dtype, lv, rv, o);
        }));
  });
}

int orca_hip_trait_transpose(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, size_t dim0,
                             size_t dim1, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* x = arg(b, s, "transpose");
    if (dim0 >= rank || dim1 >= rank) fail(ORCA_HIP_ERR_INTERNAL, "Invalid transpose dimensions");
    if (rank >= 2 && dtype == ORCA_HIP_F32 &&
        ((dim0 == rank - 2 && dim1 == rank - 1) || (dim0 == rank - 1 && dim1 == rank - 2))) {
      Buf* buf = materialize(b, x);
      (void)buf;
      Node* v = value_node(b, x->n, x->buf);
      if (x->tshape.empty()) {  // a view; transposing a view gives back the buffer's own layout
        v->tshape.assign(shape, shape + rank);
        std::swap(v->tshape[dim0], v->tshape[dim1]);
      }
      put(out, v);
      return;
    }
    Ref p = plain(b, x);
    float* sp = dptr(b, p.get());
    put(out, kernel_node(b, x->n, [&](void** o) {
          return orca_hip_transpose(b->ctx, sp, shape, rank, dim0, dim1, dtype, o);
        }));
  });
}

#define TRAIT_BINARY(NAME, OPC, FN)                                                                                     \
  int orca_hip_trait_##NAME(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,  \
                            size_t rank, int dtype, orca_hip_storage** out) {                                         \
    return entry(be, [&](Backend* b) {                                                                                \
      check_out(out);                                                                                                 \
      put(out, binary(b, OPC, FN, arg(b, lhs, #NAME), arg(b, rhs, #NAME), shape, rank, dtype));                       \
    });                                                                                                               \
  }
#define TRAIT_UNARY(NAME, OPC, FN)                                                                                   \
  int orca_hip_trait_##NAME(orca_hip_backend* be, orca_hip_storage* s, const size_t* shape, size_t rank, int dtype, \
                            orca_hip_storage** out) {                                                               \
    return entry(be, [&](Backend* b) {                                                                              \
      check_out(out);                                                                                               \
      put(out, unary(b, OPC, FN, arg(b, s, #NAME), shape, rank, dtype));                                            \
    });                                                                                                             \
  }

int orca_hip_trait_add(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                       size_t rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* l = arg(b, lhs, "add");
    Node* r = arg(b, rhs, "add");
    if (is_lazy_f32(b, dtype) && same_len({l, r}))
      if (Node* x = fold_const(b, ORCA_HIP_EW_ADD, l, r)) return put(out, x);
    put(out, binary(b, ORCA_HIP_EW_ADD, orca_hip_add, l, r, shape, rank, dtype));
  });
}
TRAIT_BINARY(sub, ORCA_HIP_EW_SUB, orca_hip_sub)

int orca_hip_trait_mul_scalar(orca_hip_backend* be, orca_hip_storage* s, float scalar, const size_t* shape, size_t rank,
                              int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* x = arg(b, s, "mul_scalar");
    if (is_lazy_f32(b, dtype)) {
      if (Node* c = const_src(x)) {
        volatile float cv = c->cval, f = scalar;
        const float v = cv * f;
        if (!std::isnan(v)) return put(out, const_node(b, v, x->n));
      }
      std::vector<Ref> o;
      o.emplace_back(ref(x));
      return put(out, ew(b, ORCA_HIP_EW_MUL_SCALAR, std::move(o), x->n, scalar));
    }
    Ref p = plain(b, x);
    float* sp = dptr(b, p.get());
    put(out, kernel_node(b, numel_of(shape, rank), [&](void** o) {
          return orca_hip_mul_scalar(b->ctx, sp, scalar, shape, rank, dtype, o);
        }));
  });
}

int orca_hip_trait_mul(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs, const size_t* shape,
                       size_t rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* l = arg(b, lhs, "mul");
    Node* r = arg(b, rhs, "mul");
    if (is_lazy_f32(b, dtype) && same_len({l, r}))
      if (Node* x = fold_const(b, ORCA_HIP_EW_MUL, l, r)) return put(out, x);
    put(out, binary(b, ORCA_HIP_EW_MUL, orca_hip_mul, l, r, shape, rank, dtype));
  });
}
TRAIT_UNARY(relu, ORCA_HIP_EW_RELU, orca_hip_relu)
TRAIT_UNARY(sigmoid, ORCA_HIP_EW_SIGMOID, orca_hip_sigmoid)
TRAIT_BINARY(relu_backward, ORCA_HIP_EW_RELU_BW, orca_hip_relu_backward)
TRAIT_BINARY(sigmoid_backward, ORCA_HIP_EW_SIGMOID_BW, orca_hip_sigmoid_backward)

int orca_hip_trait_expand(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                          const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* x = arg(b, s, "expand");
    if (dtype == ORCA_HIP_F32 && in_rank == out_rank && std::equal(in_shape, in_shape + in_rank, out_shape))
      return put(out, ref(x));  // identity broadcast: share the storage
    const size_t n = numel_of(out_shape, out_rank);
    if (is_lazy_f32(b, dtype) && out_rank >= in_rank && n > 0 && x->n == numel_of(in_shape, in_rank)) {
      if (Node* c = const_src(x)) {
        std::vector<Ref> o;
        o.emplace_back(bcast(b, c, n, 1, 1));
        return put(out, ew(b, ORCA_HIP_EW_COPY, std::move(o), n));
      }
      uint64_t dv, md;
      if (broadcast_map(in_shape, in_rank, out_shape, out_rank, &dv, &md)) {
        Ref p = plain(b, x);
        std::vector<Ref> o;
        o.emplace_back(bcast(b, p.get(), n, dv, md));
        return put(out, ew(b, ORCA_HIP_EW_COPY, std::move(o), n));
      }
    }
    put(out, reshape_like(b, orca_hip_expand, x, in_shape, in_rank, out_shape, out_rank, dtype));
  });
}

int orca_hip_trait_sum_to_shape(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                                const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* x = arg(b, s, "sum_to_shape");
    const bool no_fill = x->kind != Kind::kProd && x->kind != Kind::kColsum && x->kind != Kind::kConst;
    if (b->opt.deferred && dtype == ORCA_HIP_F32 && x->tshape.empty() && no_fill) {
      const bool same = in_rank == out_rank && std::equal(in_shape, in_shape + in_rank, out_shape);
      if (same) {  // computed once per storage (storages are immutable)
        if (x->kind == Kind::kValue && x->canon) return put(out, ref(x));
        if (x->ident) return put(out, ref(x->ident));
        Node* r;
        if (b->opt.lazy) {
          std::vector<Ref> o;
          o.emplace_back(ref(x));
          r = ew(b, ORCA_HIP_EW_SUM_VISIT, std::move(o), x->n);
        } else {
          r = reshape_like(b, orca_hip_sum_to_shape, x, in_shape, in_rank, out_shape, out_rank, dtype);
        }
        x->ident = r;
        r->ident_of = x;
        return put(out, r);
      }
      const bool row = in_rank == 2 && ((out_rank == 2 && out_shape[0] == 1 && out_shape[1] == in_shape[1]) ||
                                        (out_rank == 1 && out_shape[0] == in_shape[1]));
      if (row) return put(out, deferred_colsum(b, x, in_shape[0], in_shape[1]));
      const bool per_row = in_rank == 2 && out_rank == 2 && out_shape[0] == in_shape[0] && out_shape[1] == 1;
      if (per_row && b->opt.lazy)
        if (Node* r = chain_rows(b, x, in_shape[0], in_shape[1], false)) return put(out, r);
    }
    put(out, reshape_like(b, orca_hip_sum_to_shape, x, in_shape, in_rank, out_shape, out_rank, dtype));
  });
}

int orca_hip_trait_reshape(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                           const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* x = arg(b, s, "reshape");
    const size_t ni = numel_of(in_shape, in_rank), no = numel_of(out_shape, out_rank);
    if (ni != no) fail_shape("reshape", std::to_string(ni) + " elements", std::to_string(no) + " elements");
    (void)dtype;
    put(out, plain(b, x).release());
  });
}

TRAIT_UNARY(exp, ORCA_HIP_EW_EXP, orca_hip_exp)
TRAIT_UNARY(log, ORCA_HIP_EW_LOG, orca_hip_log)
TRAIT_BINARY(exp_backward, ORCA_HIP_EW_EXP_BW, orca_hip_exp_backward)
TRAIT_BINARY(log_backward, ORCA_HIP_EW_LOG_BW, orca_hip_log_backward)
TRAIT_BINARY(div, ORCA_HIP_EW_DIV, orca_hip_div)
TRAIT_UNARY(sqrt, ORCA_HIP_EW_SQRT, orca_hip_sqrt)
TRAIT_BINARY(div_backward_lhs, ORCA_HIP_EW_DIV, orca_hip_div_backward_lhs)

int orca_hip_trait_div_backward_rhs(orca_hip_backend* be, orca_hip_storage* grad, orca_hip_storage* lhs,
                                    orca_hip_storage* rhs, const size_t* shape, size_t rank, int dtype,
                                    orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* g = arg(b, grad, "div_backward_rhs");
    Node* l = arg(b, lhs, "div_backward_rhs");
    Node* r = arg(b, rhs, "div_backward_rhs");
    if (is_lazy_f32(b, dtype) && same_len({g, l, r})) {
      std::vector<Ref> o;
      o.emplace_back(ref(g));
      o.emplace_back(ref(l));
      o.emplace_back(ref(r));
      return put(out, ew(b, ORCA_HIP_EW_DIV_BW_RHS, std::move(o), g->n));
    }
    Ref pg = plain(b, g), pl = plain(b, l), pr = plain(b, r);
    float *gp = dptr(b, pg.get()), *lp = dptr(b, pl.get()), *rp = dptr(b, pr.get());
    put(out, kernel_node(b, numel_of(shape, rank), [&](void** o) {
          return orca_hip_div_backward_rhs(b->ctx, gp, lp, rp, shape, rank, dtype, o);
        }));
  });
}

TRAIT_BINARY(sqrt_backward, ORCA_HIP_EW_SQRT_BW, orca_hip_sqrt_backward)

int orca_hip_trait_accumulate_grad(orca_hip_backend* be, orca_hip_storage* lhs, orca_hip_storage* rhs,
                                   orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* l = arg(b, lhs, "accumulate_grad");
    Node* r = arg(b, rhs, "accumulate_grad");
    if (is_lazy_f32(b, ORCA_HIP_F32) && same_len({l, r})) {
      if (Node* x = fold_const(b, ORCA_HIP_EW_ADD, l, r)) return put(out, x);
      std::vector<Ref> o;
      o.emplace_back(ref(l));
      o.emplace_back(ref(r));
      return put(out, ew(b, ORCA_HIP_EW_ADD, std::move(o), l->n));
    }
    Ref pl = plain(b, l), pr = plain(b, r);
    float *lp = dptr(b, pl.get()), *rp = dptr(b, pr.get());
    put(out, kernel_node(b, pl->n, [&](void** o) { return orca_hip_accumulate_grad(b->ctx, lp, rp, pl->n, o); }));
  });
}

int orca_hip_trait_conv2d(orca_hip_backend* be, orca_hip_storage*, orca_hip_storage*, orca_hip_storage*,
                          const size_t*, size_t, const size_t*, size_t, size_t, size_t, size_t, size_t, int dtype,
                          orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("conv2d (hip)", dtype); });
}
int orca_hip_trait_conv2d_backward_input(orca_hip_backend* be, orca_hip_storage*, orca_hip_storage*, const size_t*,
                                         size_t, const size_t*, size_t, size_t, size_t, size_t, size_t, int dtype,
                                         orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("conv2d_backward_input (hip)", dtype); });
}
int orca_hip_trait_conv2d_backward_weight(orca_hip_backend* be, orca_hip_storage*, orca_hip_storage*, const size_t*,
                                          size_t, const size_t*, size_t, size_t, size_t, size_t, size_t, int dtype,
                                          orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("conv2d_backward_weight (hip)", dtype); });
}
int orca_hip_trait_conv2d_backward_bias(orca_hip_backend* be, orca_hip_storage*, const size_t*, size_t, int dtype,
                                        orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("conv2d_backward_bias (hip)", dtype); });
}

int orca_hip_trait_cast(orca_hip_backend* be, orca_hip_storage* s, const size_t*, size_t, int current_dtype,
                        int target_dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* x = arg(b, s, "cast");
    if (current_dtype != ORCA_HIP_F32) unsupported("cast (hip)", current_dtype);
    if (target_dtype != ORCA_HIP_F32) unsupported("cast (hip)", target_dtype);
    put(out, ref(x));
  });
}

int orca_hip_trait_scatter(orca_hip_backend* be, orca_hip_storage*, size_t, orca_hip_storage*, orca_hip_storage*,
                           const size_t*, size_t, const size_t*, size_t, int dtype, orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("scatter (hip)", dtype); });
}
int orca_hip_trait_gather(orca_hip_backend* be, orca_hip_storage*, size_t, orca_hip_storage*, const size_t*, size_t,
                          const size_t*, size_t, int dtype, orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("gather (hip)", dtype); });
}
int orca_hip_trait_scatter_backward_src(orca_hip_backend* be, orca_hip_storage*, size_t, orca_hip_storage*,
                                        const size_t*, size_t, const size_t*, size_t, int dtype, orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("scatter_backward_src (hip)", dtype); });
}
int orca_hip_trait_scatter_backward_base(orca_hip_backend* be, orca_hip_storage*, size_t, orca_hip_storage*,
                                         const size_t*, size_t, const size_t*, size_t, int dtype, orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("scatter_backward_base (hip)", dtype); });
}
int orca_hip_trait_gather_backward(orca_hip_backend* be, orca_hip_storage*, size_t, orca_hip_storage*, const size_t*,
                                   size_t, const size_t*, size_t, int dtype, orca_hip_storage**) {
  return entry(be, [&](Backend*) { unsupported("gather_backward (hip)", dtype); });
}

int orca_hip_trait_from_bytes(orca_hip_backend* be, const size_t* shape, size_t rank, const uint8_t* bytes,
                              size_t n_bytes, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    put(out, kernel_node(b, numel_of(shape, rank), [&](void** o) {
          return orca_hip_from_bytes(b->ctx, shape, rank, bytes, n_bytes, dtype, o);
        }));
  });
}

int orca_hip_trait_to_bytes(orca_hip_backend* be, orca_hip_storage* s, uint8_t* host, size_t n_bytes) {
  return entry(be, [&](Backend* b) {
    Ref p = plain(b, arg(b, s, "to_bytes"));
    if (n_bytes != 4 * p->n)
      fail_shape("to_bytes", std::to_string(4 * p->n) + " bytes", std::to_string(n_bytes) + " bytes");
    ck(orca_hip_to_bytes(b->ctx, dptr(b, p.get()), n_bytes, host));
  });
}

int orca_hip_trait_has_nan_or_inf(orca_hip_backend* be, orca_hip_storage* s, int dtype, int* result) {
  return entry(be, [&](Backend* b) {
    if (!result) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    Ref p = plain(b, arg(b, s, "has_nan_or_inf"));
    ck(orca_hip_has_nan_or_inf(b->ctx, dptr(b, p.get()), p->n, dtype, result));
  });
}

int orca_hip_trait_max_to_shape(orca_hip_backend* be, orca_hip_storage* s, const size_t* in_shape, size_t in_rank,
                                const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* x = arg(b, s, "max_to_shape");
    if (is_lazy_f32(b, dtype) && in_rank == out_rank && std::equal(in_shape, in_shape + in_rank, out_shape)) {
      std::vector<Ref> o;
      o.emplace_back(ref(x));
      return put(out, ew(b, ORCA_HIP_EW_MAX_VISIT, std::move(o), x->n));
    }
    const bool per_row = in_rank == 2 && out_rank == 2 && out_shape[0] == in_shape[0] && out_shape[1] == 1;
    if (per_row && is_lazy_f32(b, dtype) && b->opt.deferred && x->tshape.empty())
      if (Node* r = chain_rows(b, x, in_shape[0], in_shape[1], true)) return put(out, r);
    put(out, reshape_like(b, orca_hip_max_to_shape, x, in_shape, in_rank, out_shape, out_rank, dtype));
  });
}

int orca_hip_trait_max_to_shape_backward(orca_hip_backend* be, orca_hip_storage* grad, orca_hip_storage* in_primal,
                                         orca_hip_storage* out_primal, const size_t* in_shape, size_t in_rank,
                                         const size_t* out_shape, size_t out_rank, int dtype, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Ref g = plain(b, arg(b, grad, "max_to_shape_backward"));
    Ref x = plain(b, arg(b, in_primal, "max_to_shape_backward"));
    Ref y = plain(b, arg(b, out_primal, "max_to_shape_backward"));
    float *gp = dptr(b, g.get()), *xp = dptr(b, x.get()), *yp = dptr(b, y.get());
    put(out, kernel_node(b, numel_of(in_shape, in_rank), [&](void** o) {
          return orca_hip_max_to_shape_backward(b->ctx, gp, xp, yp, in_shape, in_rank, out_shape, out_rank, dtype, o);
        }));
  });
}

// ---------------------------------------------------------------- beside the trait
int orca_hip_be_softmax_ce(orca_hip_backend* be, orca_hip_storage* logits, orca_hip_storage* onehot, size_t B, size_t C,
                           int want_grad, orca_hip_storage** loss, orca_hip_storage** dlogits) {
  return entry(be, [&](Backend* b) {
    check_out(loss);
    if (want_grad) check_out(dlogits);
    Ref lg = plain(b, arg(b, logits, "softmax_ce logits"));
    Ref oh = plain(b, arg(b, onehot, "softmax_ce targets"));
    if (lg->n != B * C || oh->n != B * C)
      fail_shape("softmax_ce", std::to_string(B * C) + " elements",
                 std::to_string(lg->n) + " and " + std::to_string(oh->n) + " elements");
    float* lp = dptr(b, lg.get());
    float* op = dptr(b, oh.get());
    Ref l(value_node(b, 1, alloc_buf(b, 1)));
    Ref d;
    if (want_grad) d = Ref(value_node(b, B * C, alloc_buf(b, B * C)));
    ck(orca_hip_softmax_ce(b->ctx, lp, B, C, op, nullptr, l->buf->ptr, want_grad ? d->buf->ptr : nullptr, nullptr,
                           nullptr));
    l->quiet = true;
    // every element of the gradient is (0 + a) + (0 + b), plus (0 + c) at a row's maximum:
    // never -0, never a signaling NaN
    if (want_grad) d->quiet = d->canon = true;
    *loss = S_(l.release());
    if (want_grad) *dlogits = S_(d.release());
  });
}

int orca_hip_be_clone(orca_hip_backend* be, orca_hip_storage* s, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Ref p = plain(b, arg(b, s, "clone"));
    Ref c(value_node(b, p->n, alloc_buf(b, p->n)));
    if (p->n) ck(orca_hip_d2d(b->ctx, c->buf->ptr, dptr(b, p.get()), 4 * p->n));
    put(out, c.release());
  });
}

int orca_hip_be_arena(orca_hip_backend* be, size_t n, int fill, float value, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Ref a(value_node(b, n, alloc_buf(b, n)));
    if (fill && n) ck(orca_hip_fill(b->ctx, a->buf->ptr, value, n));
    put(out, a.release());
  });
}

int orca_hip_be_view(orca_hip_backend* be, orca_hip_storage* arena, size_t offset, size_t n, orca_hip_storage** out) {
  return entry(be, [&](Backend* b) {
    check_out(out);
    Node* a = arg(b, arena, "view");
    Buf* ab = materialize(b, a);
    if (!a->tshape.empty() || offset + n > a->n)
      fail_shape("view", "at most " + std::to_string(a->n) + " elements", std::to_string(offset + n) + " elements");
    auto v = std::make_shared<Buf>();
    v->ctx = b->ctx;
    v->ptr = ab->ptr + offset;
    v->bytes = 4 * n;
    v->owner = a->buf;
    put(out, value_node(b, n, v));
  });
}

int orca_hip_be_copy_into(orca_hip_backend* be, orca_hip_storage* dst, orca_hip_storage* src) {
  return entry(be, [&](Backend* b) {
    Node* d = arg(b, dst, "copy_into");
    Ref s = plain(b, arg(b, src, "copy_into"));
    if (s->n != d->n) fail_shape("copy_into", std::to_string(d->n) + " elements", std::to_string(s->n) + " elements");
    d->in_place = true;
    if (s->n) ck(orca_hip_d2d(b->ctx, dptr(b, d), dptr(b, s.get()), 4 * s->n));
  });
}

int orca_hip_be_arena_exclusive(orca_hip_backend* be, orca_hip_storage* arena, int* exclusive) {
  return entry(be, [&](Backend* b) {
    if (!exclusive) fail(ORCA_HIP_ERR_INTERNAL, "null output pointer");
    Node* a = arg(b, arena, "arena_exclusive");
    // the caller's handle is the only reference to the node, and the node the only holder of
    // its memory (every view, and every storage sharing it, holds the buffer)
    *exclusive = a->rc.load() == 1 && a->buf && a->buf.use_count() == 1 ? 1 : 0;
  });
}

static int opt_multi(orca_hip_backend* be, const orca_hip_opt_row* rows, size_t n_rows, bool adamw, double lr,
                     double b1, double b2, double eps, double wd, int64_t t) {
  return entry(be, [&](Backend* b) {
    if (n_rows && !rows) fail(ORCA_HIP_ERR_INTERNAL, "null row array");
    std::vector<Row> rs;
    std::vector<Ref> plains;  // materialised transposes of p_src / g
    for (size_t i = 0; i < n_rows; ++i) {
      const orca_hip_opt_row& r = rows[i];
      Row x{};
      plains.push_back(plain(b, arg(b, r.p_src, "optimizer p_src")));
      x.p_src = plains.back().get();
      x.p_dst = arg(b, r.p_dst, "optimizer p_dst");
      plains.push_back(plain(b, arg(b, r.g, "optimizer gradient")));
      x.g = plains.back().get();
      if (adamw) {
        x.m = arg(b, r.m, "optimizer m");
        x.v = arg(b, r.v, "optimizer v");
      }
      x.n = r.n;
      rs.push_back(x);
    }
    std::vector<Node*> written;
    for (auto& r : rs) {
      written.push_back(r.p_dst);
      if (adamw) {
        written.push_back(r.m);
        written.push_back(r.v);
      }
    }
    // the update changes these in place: what was derived from them is computed first
    mutating(b, written);
    auto launch = [&](const std::vector<PtrRow>& ptrs) {
      for (size_t from = 0; from < ptrs.size(); from += ORCA_HIP_OPT_MAX_SEGMENTS) {
        const size_t cnt = std::min<size_t>(ORCA_HIP_OPT_MAX_SEGMENTS, ptrs.size() - from);
        auto segs = segments(ptrs, from, cnt);
        if (adamw)
          ck(orca_hip_adamw_multi(b->ctx, segs.data(), segs.size(), lr, b1, b2, eps, wd, t));
        else
          ck(orca_hip_sgd_multi(b->ctx, segs.data(), segs.size(), lr));
      }
    };
    optimizer_pass(b, rs, adamw, launch);
  });
}

int orca_hip_be_adamw_multi(orca_hip_backend* be, const orca_hip_opt_row* rows, size_t n_rows, double lr, double beta1,
                            double beta2, double eps, double weight_decay, int64_t t) {
  return opt_multi(be, rows, n_rows, true, lr, beta1, beta2, eps, weight_decay, t);
}

int orca_hip_be_sgd_multi(orca_hip_backend* be, const orca_hip_opt_row* rows, size_t n_rows, double lr) {
  return opt_multi(be, rows, n_rows, false, lr, 0, 0, 0, 0, 0);
}

int orca_hip_be_adamw_step(orca_hip_backend* be, orca_hip_storage* p, orca_hip_storage* g, orca_hip_storage* m,
                           orca_hip_storage* v, size_t n, double lr, double beta1, double beta2, double eps,
                           double weight_decay, int64_t t) {
  return entry(be, [&](Backend* b) {
    Node *pp = arg(b, p, "adamw_step p"), *mm = arg(b, m, "adamw_step m"), *vv = arg(b, v, "adamw_step v");
    Ref gg = plain(b, arg(b, g, "adamw_step g"));
    float* gp = dptr(b, gg.get());
    mutating(b, std::vector<Node*>{pp, mm, vv});
    ck(orca_hip_adamw_step(b->ctx, dptr(b, pp), gp, dptr(b, mm), dptr(b, vv), n, lr, beta1, beta2, eps, weight_decay,
                           t));
  });
}

int orca_hip_be_sgd_step(orca_hip_backend* be, orca_hip_storage* p, orca_hip_storage* g, size_t n, double lr) {
  return entry(be, [&](Backend* b) {
    Node* pp = arg(b, p, "sgd_step p");
    Ref gg = plain(b, arg(b, g, "sgd_step g"));
    float* gp = dptr(b, gg.get());
    mutating(b, std::vector<Node*>{pp});
    ck(orca_hip_sgd_step(b->ctx, dptr(b, pp), gp, n, lr));
  });
}

}  // extern "C"
