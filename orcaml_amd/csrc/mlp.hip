// Device-resident training step of nn.Sequential(Linear, ReLU, ..., Linear)
// + CrossEntropyLoss + SGD/AdamW (python/orca/nn/{linear,activation,
// container,loss}.py, python/orca/optim/{sgd,adamw}.py).
//
// HBM layout: parameters, gradients and the AdamW moments live in four flat
// arenas with one common layout, [W_0 | b_0 | W_1 | b_1 | ...], each tensor
// starting on a 256-byte boundary (padding is zero in every arena and stays
// zero under both updates).  Activations keep only the ReLU outputs: the
// mask of ReluBackward ([pre > 0], orca-backend-cpu/src/backend.rs:434)
// equals [relu(pre) > 0].  A step is, for L layers:
//   forward   L GEMMs  (bias + ReLU fused into the epilogue; bias only on the last)
//   loss      fused softmax-CE forward/gradient/argmax + a one-block finish
//   backward  L GEMMs dW = A^T dZ with the bias column sum fused in, and
//             L-1 GEMMs dZ_prev = (dZ W^T) * [H > 0] with the mask fused in
//   update    one AdamW or SGD pass over the whole parameter arena.
// When the last layer has at most 16 outputs (a classifier), its three
// products and the loss are HBM-bound rather than GEMM-shaped; they run as
// the two fused head kernels instead (forward + loss, and backward), each
// streaming the layer's input once.  ORCA_HIP_FUSED_HEAD=0 at creation keeps
// the GEMM + softmax-CE path, ORCA_HIP_OVERLAP_UPDATE=0 runs the whole update
// on the context stream after the backward (A/B comparisons).
// With AdamW and a side stream the parameters have two arenas, P and P_next:
// the update reads P and writes P_next, and they swap after each step.  The
// update of layers >= 1 then starts right after dW of layer 1, beside layer
// 1's dZ product (which reads P): 70 % of it on a grid of two blocks per CU
// (room for the GEMM's blocks), the rest on the flat grid once that product
// is done, beside layer 0's dW.  ORCA_HIP_DOUBLE_ARENA=0 keeps one arena;
// ORCA_HIP_SIDE_FRAC (percent) and ORCA_HIP_SIDE_BPC tune the split.
// Every buffer, split-K workspaces included, is allocated at creation: a step
// allocates nothing and never synchronises.  With ORCA_HIP_GRAPH=1 the step is
// captured into a HIP graph at its first call (forward, loss, backward and the
// optimizer passes on both streams) and replayed; the only per-step host work
// is then one launch storing the step's AdamW scalars, which the graph reads
// from device memory.
#include <cstdlib>
#include <cstring>
#include <vector>

#include "runtime.hpp"

struct orca_hip_mlp {
  orca_hip_ctx* ctx = nullptr;
  std::vector<size_t> dims;
  size_t L = 0, B = 0;
  orca_hip_optim opt{};
  int64_t t = 0;
  std::vector<size_t> off;  // arena offset of parameter i (floats)
  std::vector<size_t> cnt;  // element count of parameter i
  size_t arena = 0;         // arena length (floats)
  float *P = nullptr, *G = nullptr, *Mo = nullptr, *Vo = nullptr;
  float* x = nullptr;
  float* onehot = nullptr;
  int32_t* labels = nullptr;
  std::vector<float*> H;   // ReLU outputs of layers 0..L-2
  float* logits = nullptr;
  float* dlogits = nullptr;
  float* dz[2] = {nullptr, nullptr};
  float* loss = nullptr;
  int64_t* correct = nullptr;
  int32_t* preds = nullptr;
  std::vector<void*> owned;
  bool have_batch = false;
  bool fused_head = false;
  // With the fused head, its backward kernel also sums dZ of the layer below over the
  // rows (that layer's bias gradient), so that layer's dW product runs without the
  // folded column sum (ORCA_HIP_HEAD_DB=0 keeps the fold).
  bool head_db = false;
  orca_hip::HeadWorkspace head;
  // Second stream (default priority) for the update of layers >= 1, which
  // overlaps the first layer's weight-gradient GEMM; fork / join events.
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr, mid = nullptr;
  // Second parameter arena: with it, AdamW reads P and writes P_next, so the
  // update of layers >= 1 can start as soon as their gradients exist (dW of
  // layer 1) and run beside layer 1's dZ product, which still reads P; the
  // two arenas swap roles after every step.
  float* P_next = nullptr;
  // The side-stream update in two parts: [split, split + side_a) with a grid of
  // side_bpc blocks per CU beside layer 1's dZ product, the rest with the flat
  // grid once that product is done (beside layer 0's dW, which leaves CUs idle).
  int side_bpc = 2;
  // The update of layer 0 (after its dW, alone on the GPU) on 8 blocks per CU, each thread
  // keeping several float4 groups of each array in flight: 15.2 against 16.0 us on the flat
  // grid for 784-4096 (ORCA_HIP_U0_BPC; 0 = the flat grid).
  int u0_bpc = 8;
  // fork / mid events bound to the completion of the GEMM before them
  bool bind_events = true;
  size_t side_a = 0;
  // The second side part [split + side_a, split + side_a + side_b) beside layer 0's
  // dW on side_bpc2 blocks per CU (0 = the flat grid); what is left of the arena
  // after it is updated on the context stream after that product, with layer 0.
  size_t side_b = 0;
  int side_bpc2 = 0;
  // One rank's share of a data-parallel step whose optimizer state is sharded over
  // shard_count ranks.  The rank owns slice shard_index (cuts at multiples of 64 floats) of
  // each range between consecutive shard_cuts: layer 0, then the parts of layers >= 1 that
  // the double-arena schedule updates beside layer 1's dZ product, beside layer 0's dW and
  // after it.  That map is fixed for the model, whatever schedule a step takes (captured or
  // not, second stream or not), and every rank does the same work.  Each update pass covers
  // its range's intersection with the owned slices; a slice of layers >= 1 too small for the
  // second stream (kMinShardOverlapParams) updates with layer 0's after the backward.  The
  // other slices keep their values in both arenas.
  size_t shard_index = 0, shard_count = 1;
  std::vector<size_t> shard_cuts;
  // Persistent workspaces: a step makes no allocator call, so it can be
  // captured once into a HIP graph and replayed.
  orca_hip::AdamWScalars* kdev = nullptr;  // this step's AdamW scalars (device)
  float* gemm_ws = nullptr;                // split-K partials of the step's GEMMs
  size_t gemm_ws_floats = 0;
  bool use_graph = false;
  hipGraphExec_t exec = nullptr;

  float* dev(size_t n) {
    void* p = orca_hip::ctx_allocate(ctx, n * sizeof(float) + 256);
    owned.push_back(p);
    return static_cast<float*>(p);
  }
  ~orca_hip_mlp() {
    if (exec) (void)hipGraphExecDestroy(exec);
    for (void* p : owned) ctx->alloc.release(p);
    if (fork) (void)hipEventDestroy(fork);
    if (join) (void)hipEventDestroy(join);
    if (mid) (void)hipEventDestroy(mid);
    if (side) (void)hipStreamDestroy(side);
  }
};

namespace orca_hip {
namespace {

// The fork / mid / join events order the two streams on this device only: no
// system-scope fence at record (the kernels' own release and acquire are at
// device scope).  Measured: 0.9163 -> 0.9102 ms per step (median of 6 x 100).
constexpr unsigned kStreamEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;

// Smallest update (parameters of layers >= 1) worth a second stream.
constexpr size_t kMinOverlapParams = size_t(1) << 22;
// The same for one rank's slice of a sharded update: on 784-4096-4096-10 the second stream paid
// at 8.4 M parameters per rank (512 rows, 2 ranks: 0.518 against 0.520 ms per step) and not at
// 4.2 M (256 rows, 4 ranks: 0.306 against 0.302) or 2.1 M (128 rows, 8 ranks: 0.204 against
// 0.194), where the whole slice runs after the backward on the context stream instead.
constexpr size_t kMinShardOverlapParams = size_t(6) << 20;

// Everything a step enqueues.  With kdev set, AdamW reads its scalars from
// that device buffer, so the enqueued work is identical from step to step and
// is what a captured graph replays; without it they are kernel arguments.
void step_body(orca_hip_mlp* m, const AdamWScalars* kdev) {
  orca_hip_ctx* ctx = m->ctx;
  const size_t L = m->L, B = m->B, C = m->dims[L];
  const size_t n_gemm = m->fused_head ? L - 1 : L;  // layers run as GEMMs
  // ---- forward ----
  for (size_t l = 0; l < n_gemm; ++l) {
    const size_t K = m->dims[l], N = m->dims[l + 1];
    const float* a = l == 0 ? m->x : m->H[l - 1];
    GemmEpi e;
    e.ws = m->gemm_ws;
    e.ws_floats = m->gemm_ws_floats;
    e.kind = l + 1 < L ? ORCA_HIP_EPI_BIAS_RELU : ORCA_HIP_EPI_BIAS;
    e.bias = m->P + m->off[2 * l + 1];
    float* out = l + 1 < L ? m->H[l] : m->logits;
    gemm(ctx, false, false, B, N, K, a, K, 0, m->P + m->off[2 * l], N, 0, out, N, 0, 1, e);
  }
  // ---- loss and its gradient (with the last layer when it is a fused head) ----
  const int32_t* labels = m->onehot ? nullptr : m->labels;
  if (m->fused_head) {
    const size_t l = L - 1;
    head_forward(ctx, l == 0 ? m->x : m->H[l - 1], B, m->dims[l], m->P + m->off[2 * l], m->P + m->off[2 * l + 1], C,
                 m->onehot, labels, m->logits, m->dlogits, m->preds, m->head);
  } else {
    softmax_ce(ctx, m->logits, B, C, m->onehot, labels, m->loss, m->dlogits, m->preds, m->correct,
               m->head.row_loss, m->head.row_correct);
  }
  // ---- backward ----
  const float* g = m->dlogits;
  int ping = 0;
  if (m->fused_head) {
    const size_t l = L - 1;
    float* dz = l > 0 ? m->dz[ping] : nullptr;
    // The backward kernel also adds the forward's row terms into the loss.
    head_backward(ctx, l == 0 ? m->x : m->H[l - 1], B, m->dims[l], m->P + m->off[2 * l], C, m->dlogits, l > 0, dz,
                  m->G + m->off[2 * l], m->G + m->off[2 * l + 1], &m->head, m->loss, m->correct,
                  dz && m->head_db ? m->G + m->off[2 * (l - 1) + 1] : nullptr);
    if (dz) {
      g = dz;
      ping ^= 1;
    }
  }
  // Layers >= 1 are final once the GEMMs of layer 1 have run: their gradients
  // are complete and no later kernel of the step reads their weights.  With
  // a side stream, their update then runs concurrently with layer 0's
  // weight-gradient GEMM (memory-bound beside compute-bound); the step ends
  // when both streams have finished.
  const size_t split = L > 1 ? m->off[2] : 0;  // arena offset of W_1
  // whether this step's update of layers >= 1 runs on the second stream
  const bool overlap = m->side && split > 0 &&
                       (m->shard_count == 1 || (m->arena - split) / m->shard_count >= kMinShardOverlapParams);
  bool forked = false;
  // With a second arena the update writes P_next and reads P.
  float* P_out = m->P_next ? m->P_next : m->P;
  auto update_range = [&](size_t begin, size_t end, hipStream_t stream, int bpc) {
    if (m->opt.kind == 1)
      adamw(ctx, P_out + begin, m->G + begin, m->Mo + begin, m->Vo + begin, end - begin, m->opt.lr, m->opt.beta1,
            m->opt.beta2, m->opt.eps, m->opt.weight_decay, m->t, stream, kdev, m->P + begin, bpc);
    else
      sgd(ctx, m->P + begin, m->G + begin, end - begin, m->opt.lr, stream);
  };
  auto update = [&](size_t begin, size_t end, hipStream_t stream, int bpc = 0) {
    if (end <= begin) return;
    if (m->shard_count > 1) {  // the pass's intersection with this rank's slices
      const std::vector<size_t>& cu = m->shard_cuts;
      const size_t s = m->shard_index, c = m->shard_count;
      for (size_t r = 0; r + 1 < cu.size(); ++r) {
        const size_t len = cu[r + 1] - cu[r];
        auto cut = [&](size_t i) { return i == c ? len : len * i / c / 64 * 64; };
        const size_t lo = std::max(begin, cu[r] + cut(s)), hi = std::min(end, cu[r] + cut(s + 1));
        if (lo < hi) update_range(lo, hi, stream, bpc);
      }
      return;
    }
    update_range(begin, end, stream, bpc);
  };
  auto fork_update = [&]() {
    ORCA_HIP_CHECK(hipEventRecord(m->fork, ctx->stream));
    ORCA_HIP_CHECK(hipStreamWaitEvent(m->side, m->fork, 0));
    update(split, m->arena, m->side);
    ORCA_HIP_CHECK(hipEventRecord(m->join, m->side));
    forked = true;
  };
  for (size_t l = n_gemm; l-- > 0;) {
    const size_t K = m->dims[l], N = m->dims[l + 1];
    const float* a = l == 0 ? m->x : m->H[l - 1];
    if (l == 0 && overlap && !forked) fork_update();
    GemmEpi ew;
    ew.ws = m->gemm_ws;
    ew.ws_floats = m->gemm_ws_floats;
    // bias gradient (the head's backward kernel already summed the layer below it)
    ew.colsum = m->head_db && l + 2 == L ? nullptr : m->G + m->off[2 * l + 1];
    // Layers >= 1 have all their gradients after dW of layer 1; with a second
    // arena nothing of this step writes the P that layer 1's dZ reads.
    const bool early = l == 1 && m->P_next && overlap;
    // Layer 0's weight gradient has the update of the layers above beside it when there
    // is a side stream: its banded grid then leaves CUs free for that update.
    // The form follows the model (a second stream or not), not the step's schedule, so that a
    // sharded step runs the whole step's dW bits (the two forms round differently).
    if (l == 0) ew.band = m->side ? 2 : 1;
    // The fork and mid events complete with the product's kernel rather than
    // as markers of their own between two launches.
    if (early && m->bind_events) ew.done = m->fork;
    gemm(ctx, true, false, K, N, B, a, K, 0, g, N, 0, m->G + m->off[2 * l], N, 0, 1, ew);
    if (early) {
      if (!ew.done) ORCA_HIP_CHECK(hipEventRecord(m->fork, ctx->stream));
      ORCA_HIP_CHECK(hipStreamWaitEvent(m->side, m->fork, 0));
      update(split, split + m->side_a, m->side, m->side_bpc);
      forked = true;
    }
    if (l > 0) {
      GemmEpi ex;
      ex.ws = m->gemm_ws;
      ex.ws_floats = m->gemm_ws_floats;
      ex.kind = ORCA_HIP_EPI_RELU_MASK;
      ex.mask = m->H[l - 1];
      ex.ldmask = K;
      float* dz = m->dz[ping];
      if (early && m->bind_events) ex.done = m->mid;
      gemm(ctx, false, true, B, K, N, g, N, 0, m->P + m->off[2 * l], N, 0, dz, K, 0, 1, ex);
      g = dz;
      ping ^= 1;
    }
    if (early) {
      if (!m->bind_events) ORCA_HIP_CHECK(hipEventRecord(m->mid, ctx->stream));
      ORCA_HIP_CHECK(hipStreamWaitEvent(m->side, m->mid, 0));
      update(split + m->side_a, split + m->side_a + m->side_b, m->side, m->side_bpc2);
      ORCA_HIP_CHECK(hipEventRecord(m->join, m->side));
    }
  }
  // ---- update (parameter order W_0, b_0, W_1, ...; flat passes over the arena) ----
  if (forked) {
    update(0, split, ctx->stream, m->u0_bpc);
    if (m->P_next) update(split + m->side_a + m->side_b, m->arena, ctx->stream, m->u0_bpc);
    ORCA_HIP_CHECK(hipStreamWaitEvent(ctx->stream, m->join, 0));
  } else {
    update(0, m->arena, ctx->stream);
  }
}

// Captures step_body into m->exec (the stream leaves capture mode on failure).
void capture(orca_hip_mlp* m) {
  hipStream_t s = m->ctx->stream;
  ORCA_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  try {
    step_body(m, m->kdev);
  } catch (...) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(s, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  hipGraph_t g = nullptr;
  ORCA_HIP_CHECK(hipStreamEndCapture(s, &g));
  const hipError_t e = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) m->exec = nullptr;
  ORCA_HIP_CHECK(e);
}

void invalidate_graph(orca_hip_mlp* m) {
  if (m->exec) ORCA_HIP_CHECK(hipGraphExecDestroy(m->exec));
  m->exec = nullptr;
}

void step(orca_hip_mlp* m) {
  orca_hip_ctx* ctx = m->ctx;
  if (m->opt.kind == 1) m->t += 1;
  // Per-kernel timing needs events around each launch: run eagerly then.
  if (!m->use_graph || ctx->prof.enabled) {
    step_body(m, nullptr);
    if (m->P_next) std::swap(m->P, m->P_next);
    return;
  }
  if (m->opt.kind == 1)
    adamw_store_scalars(ctx, m->kdev,
                        adamw_scalars(m->opt.lr, m->opt.beta1, m->opt.beta2, m->opt.eps, m->opt.weight_decay, m->t),
                        ctx->stream);
  if (!m->exec) capture(m);
  ORCA_HIP_CHECK(hipGraphLaunch(m->exec, ctx->stream));
}

orca_hip_mlp* checked(orca_hip_mlp* m) {
  if (!m) fail(ORCA_HIP_ERR_INTERNAL, "null orca_hip_mlp");
  bind(m->ctx);
  return m;
}

void check_index(const orca_hip_mlp* m, size_t index, size_t n) {
  if (index >= m->off.size())
    fail(ORCA_HIP_ERR_INTERNAL, "parameter index " + std::to_string(index) + " out of range");
  if (n != m->cnt[index])
    fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during mlp parameter copy: expected " + std::to_string(m->cnt[index]) +
                                 " elements, got " + std::to_string(n));
}

}  // namespace
}  // namespace orca_hip

using namespace orca_hip;

extern "C" {

int orca_hip_mlp_create(orca_hip_ctx* ctx, const size_t* dims, size_t n_layers, size_t batch,
                        const orca_hip_optim* opt, orca_hip_mlp** out) {
  return guard([&] {
    bind(ctx);
    if (!dims || !opt || !out) fail(ORCA_HIP_ERR_INTERNAL, "null argument");
    if (n_layers == 0 || batch == 0) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during mlp_create: empty model or batch");
    for (size_t i = 0; i <= n_layers; ++i)
      if (dims[i] == 0) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during mlp_create: zero-width layer");
    if (dims[n_layers] > 4096) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during mlp_create: at most 4096 classes");
    if (opt->kind != 0 && opt->kind != 1) fail(ORCA_HIP_ERR_INTERNAL, "unknown optimizer kind");
    auto m = std::unique_ptr<orca_hip_mlp>(new orca_hip_mlp());
    m->ctx = ctx;
    m->dims.assign(dims, dims + n_layers + 1);
    m->L = n_layers;
    m->B = batch;
    m->opt = *opt;
    size_t o = 0;
    for (size_t l = 0; l < n_layers; ++l) {
      for (size_t n : {dims[l] * dims[l + 1], dims[l + 1]}) {
        m->off.push_back(o);
        m->cnt.push_back(n);
        o += (n + 63) / 64 * 64;
      }
    }
    m->arena = o;
    m->P = m->dev(o);
    m->G = m->dev(o);
    launch_fill(ctx, m->P, 0.0f, o);
    launch_fill(ctx, m->G, 0.0f, o);
    if (opt->kind == 1) {
      m->Mo = m->dev(o);
      m->Vo = m->dev(o);
      launch_fill(ctx, m->Mo, 0.0f, o);
      launch_fill(ctx, m->Vo, 0.0f, o);
    }
    const size_t C = dims[n_layers];
    m->x = m->dev(batch * dims[0]);
    m->labels = reinterpret_cast<int32_t*>(m->dev(batch));
    size_t maxh = 1;
    for (size_t l = 1; l < n_layers; ++l) {
      m->H.push_back(m->dev(batch * dims[l]));
      maxh = std::max(maxh, dims[l]);
    }
    m->logits = m->dev(batch * C);
    m->dlogits = m->dev(batch * C);
    m->dz[0] = m->dev(batch * maxh);
    m->dz[1] = m->dev(batch * maxh);
    m->loss = m->dev(1);
    m->correct = reinterpret_cast<int64_t*>(m->dev(2));
    m->preds = reinterpret_cast<int32_t*>(m->dev(batch));
    // The fork / join costs more than it hides unless the overlapped update is
    // large (measured: it slows the 784-128-128-10 and 784-1024-1024-10 steps).
    const char* ov = std::getenv("ORCA_HIP_OVERLAP_UPDATE");
    const size_t overlapped = n_layers > 1 ? o - m->off[2] : 0;
    if (overlapped >= kMinOverlapParams && !(ov && ov[0] == '0')) {
      ORCA_HIP_CHECK(hipStreamCreateWithFlags(&m->side, hipStreamNonBlocking));
      ORCA_HIP_CHECK(hipEventCreateWithFlags(&m->fork, kStreamEventFlags));
      ORCA_HIP_CHECK(hipEventCreateWithFlags(&m->join, kStreamEventFlags));
    }
    const char* fh = std::getenv("ORCA_HIP_FUSED_HEAD");
    m->fused_head = head_supported(batch, dims[n_layers - 1], C) && !(fh && fh[0] == '0');
    const char* hd = std::getenv("ORCA_HIP_HEAD_DB");
    m->head_db = m->fused_head && n_layers > 1 && !(hd && hd[0] == '0');
    m->head.row_loss = m->dev(batch);
    m->head.row_correct = reinterpret_cast<int*>(m->dev(batch));
    if (opt->kind == 1) m->kdev = reinterpret_cast<AdamWScalars*>(m->dev(sizeof(AdamWScalars) / sizeof(float)));
    // The largest split-K workspace among the step's GEMMs (they run one after another on one stream).
    size_t ws = 0;
    const size_t n_gemm = m->fused_head ? n_layers - 1 : n_layers;
    for (size_t l = 0; l < n_gemm; ++l) {
      const size_t K = dims[l], N = dims[l + 1];
      const float* a = l == 0 ? m->x : m->H[l - 1];
      const float* g = l + 1 == n_layers ? m->dlogits : m->dz[0];
      const int f_epi = l + 1 < n_layers ? ORCA_HIP_EPI_BIAS_RELU : ORCA_HIP_EPI_BIAS;
      ws = std::max(ws, gemm_workspace_floats(ctx, false, false, batch, N, K, a, K, 0, m->P + m->off[2 * l], N, 0, 1,
                                              false, f_epi));
      ws = std::max(ws, gemm_workspace_floats(ctx, true, false, K, N, batch, a, K, 0, g, N, 0, 1, true));
      if (l > 0)
        ws = std::max(ws, gemm_workspace_floats(ctx, false, true, batch, K, N, g, N, 0, m->P + m->off[2 * l], N, 0,
                                                1, false, ORCA_HIP_EPI_RELU_MASK));
    }
    if (ws) {
      m->gemm_ws = m->dev(ws);
      m->gemm_ws_floats = ws;
    }
    // Replaying the captured step measured slower than launching its kernels
    // on this runtime (784-4096-4096-10: 1.083 against 1.000 ms per step), so
    // it is opt-in.
    const char* eg = std::getenv("ORCA_HIP_GRAPH");
    m->use_graph = eg && eg[0] == '1';
    // A captured step holds fixed arena pointers, so the second arena is for
    // eager steps with AdamW and a side stream only.
    const char* da = std::getenv("ORCA_HIP_DOUBLE_ARENA");
    // The side-stream parts of the update of layers >= 1 ([span] floats): a beside layer 1's
    // dZ product, b beside layer 0's dW.
    auto side_split = [](size_t span, size_t& a, size_t& b) {
      const char* sf = std::getenv("ORCA_HIP_SIDE_FRAC");
      const double frac = sf ? std::atof(sf) / 100.0 : 0.7;
      a = std::min(span, (size_t)(frac * (double)span) / 64 * 64);
      b = span - a;
      if (const char* sf2 = std::getenv("ORCA_HIP_SIDE_FRAC2"))
        b = std::min(b, (size_t)(std::atof(sf2) / 100.0 * (double)span) / 64 * 64);
    };
    const char* sb = std::getenv("ORCA_HIP_SIDE_BPC");
    if (sb) m->side_bpc = std::atoi(sb);
    if (const char* u0 = std::getenv("ORCA_HIP_U0_BPC")) m->u0_bpc = std::atoi(u0);
    if (const char* be = std::getenv("ORCA_HIP_BIND_EVENTS")) m->bind_events = be[0] != '0';
    if (m->side && opt->kind == 1 && !m->use_graph && !(da && da[0] == '0')) {
      m->P_next = m->dev(o);
      launch_fill(ctx, m->P_next, 0.0f, o);
      ORCA_HIP_CHECK(hipEventCreateWithFlags(&m->mid, kStreamEventFlags));
      side_split(o - m->off[2], m->side_a, m->side_b);
      if (const char* b2 = std::getenv("ORCA_HIP_SIDE_BPC2")) m->side_bpc2 = std::atoi(b2);
    }
    // The ranges a sharded update's slices are cut from: the double-arena schedule's update
    // passes, whichever schedule this trainer runs, so that a rank's slices depend on the
    // model (and the split's settings) only.
    m->shard_cuts = {0};
    if (n_layers > 1) {
      const size_t split = m->off[2];
      size_t a = m->side_a, b = m->side_b;
      if (!m->P_next) side_split(o - split, a, b);
      for (size_t cut : {split, split + a, split + a + b})
        if (cut > m->shard_cuts.back() && cut < o) m->shard_cuts.push_back(cut);
    }
    m->shard_cuts.push_back(o);
    host_sync(ctx);
    *out = m.release();
  });
}

int orca_hip_mlp_destroy(orca_hip_mlp* mlp) {
  return guard([&] {
    if (!mlp) return;
    bind(mlp->ctx);
    host_sync(mlp->ctx);
    delete mlp;
  });
}

int orca_hip_mlp_param_numel(const orca_hip_mlp* mlp, size_t index, size_t* n) {
  return guard([&] {
    if (!mlp || !n) fail(ORCA_HIP_ERR_INTERNAL, "null argument");
    if (index >= mlp->cnt.size()) fail(ORCA_HIP_ERR_INTERNAL, "parameter index out of range");
    *n = mlp->cnt[index];
  });
}

// Uploads are stream-ordered with no host wait (upload_async: a kernel argument or the
// pinned staging ring), so a checkpoint restore of every tensor waits for the device not
// once; the next step's kernels run after them on the context stream.
int orca_hip_mlp_set_param(orca_hip_mlp* mlp, size_t index, const float* host, size_t n) {
  return guard([&] {
    checked(mlp);
    check_index(mlp, index, n);
    upload_async(mlp->ctx, mlp->P + mlp->off[index], host, n * sizeof(float));
    // a sharded update writes only its slices of the second arena: the rest comes from here
    if (mlp->shard_count > 1 && mlp->P_next)
      upload_async(mlp->ctx, mlp->P_next + mlp->off[index], host, n * sizeof(float));
  });
}

int orca_hip_mlp_set_update_shard(orca_hip_mlp* mlp, size_t index, size_t count) {
  return guard([&] {
    checked(mlp);
    if (count == 0 || index >= count)
      fail(ORCA_HIP_ERR_INTERNAL, "update shard " + std::to_string(index) + " of " + std::to_string(count) +
                                      " out of range");
    // Both arenas hold the current values of the slices this share leaves alone.
    if (count > 1 && mlp->P_next)
      ORCA_HIP_CHECK(hipMemcpyAsync(mlp->P_next, mlp->P, mlp->arena * sizeof(float), hipMemcpyDeviceToDevice,
                                    mlp->ctx->stream));
    mlp->shard_index = index;
    mlp->shard_count = count;
    invalidate_graph(mlp);  // a captured step holds the passes' ranges
  });
}

static int read_arena(orca_hip_mlp* mlp, const float* arena, size_t index, float* host, size_t n) {
  return guard([&] {
    checked(mlp);
    check_index(mlp, index, n);
    if (!arena) fail(ORCA_HIP_ERR_INTERNAL, "state not present for this optimizer");
    ORCA_HIP_CHECK(hipMemcpyAsync(host, arena + mlp->off[index], n * sizeof(float), hipMemcpyDeviceToHost,
                                  mlp->ctx->stream));
    host_sync(mlp->ctx);
  });
}

int orca_hip_mlp_get_param(orca_hip_mlp* mlp, size_t index, float* host, size_t n) {
  return read_arena(mlp, mlp ? mlp->P : nullptr, index, host, n);
}

int orca_hip_mlp_get_grad(orca_hip_mlp* mlp, size_t index, float* host, size_t n) {
  return read_arena(mlp, mlp ? mlp->G : nullptr, index, host, n);
}

int orca_hip_mlp_get_moment(orca_hip_mlp* mlp, int which, size_t index, float* host, size_t n) {
  return read_arena(mlp, mlp ? (which == 0 ? mlp->Mo : mlp->Vo) : nullptr, index, host, n);
}

// Restores optimizer state from a checkpoint (the reference keeps m and v in
// Python lists, python/orca/optim/adamw.py:30-31, and never saves them).
int orca_hip_mlp_set_moment(orca_hip_mlp* mlp, int which, size_t index, const float* host, size_t n) {
  return guard([&] {
    checked(mlp);
    check_index(mlp, index, n);
    if (which != 0 && which != 1) fail(ORCA_HIP_ERR_INTERNAL, "moment index must be 0 (m) or 1 (v)");
    float* arena = which == 0 ? mlp->Mo : mlp->Vo;
    if (!arena) fail(ORCA_HIP_ERR_INTERNAL, "state not present for this optimizer");
    upload_async(mlp->ctx, arena + mlp->off[index], host, n * sizeof(float));
  });
}

int orca_hip_mlp_set_batch(orca_hip_mlp* mlp, const float* x, const float* onehot, const int32_t* labels) {
  return guard([&] {
    checked(mlp);
    if (!x || (onehot == nullptr) == (labels == nullptr))
      fail(ORCA_HIP_ERR_INTERNAL, "set_batch needs x and exactly one of one-hot targets or labels");
    const size_t B = mlp->B, C = mlp->dims[mlp->L];
    upload_async(mlp->ctx, mlp->x, x, B * mlp->dims[0] * sizeof(float));
    // The captured step bakes in which target buffer it reads.
    if ((onehot != nullptr) != (mlp->onehot != nullptr)) invalidate_graph(mlp);
    if (onehot) {
      if (!mlp->onehot) mlp->onehot = mlp->dev(B * C);
      upload_async(mlp->ctx, mlp->onehot, onehot, B * C * sizeof(float));
    } else {
      upload_async(mlp->ctx, mlp->labels, labels, B * sizeof(int32_t));
      if (mlp->onehot) {  // switch to label targets
        mlp->ctx->alloc.release(mlp->onehot);
        for (auto& p : mlp->owned)
          if (p == mlp->onehot) p = nullptr;
        mlp->owned.erase(std::remove(mlp->owned.begin(), mlp->owned.end(), nullptr), mlp->owned.end());
        mlp->onehot = nullptr;
      }
    }
    mlp->have_batch = true;
  });
}

int orca_hip_mlp_batch_ptrs(orca_hip_mlp* mlp, float** x, int32_t** labels) {
  return guard([&] {
    checked(mlp);
    if (x) *x = mlp->x;
    if (labels) *labels = mlp->labels;
  });
}

int orca_hip_mlp_step(orca_hip_mlp* mlp) {
  return guard([&] {
    checked(mlp);
    if (!mlp->have_batch) fail(ORCA_HIP_ERR_INTERNAL, "mlp_step before set_batch");
    step(mlp);
  });
}

int orca_hip_mlp_read_metrics(orca_hip_mlp* mlp, float* loss, int64_t* correct) {
  return guard([&] {
    checked(mlp);
    hipStream_t s = mlp->ctx->stream;
    if (loss) ORCA_HIP_CHECK(hipMemcpyAsync(loss, mlp->loss, sizeof(float), hipMemcpyDeviceToHost, s));
    if (correct) ORCA_HIP_CHECK(hipMemcpyAsync(correct, mlp->correct, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    host_sync(mlp->ctx, s);
  });
}

int orca_hip_mlp_get_logits(orca_hip_mlp* mlp, float* host, size_t n) {
  return guard([&] {
    checked(mlp);
    size_t want = mlp->B * mlp->dims[mlp->L];
    if (n != want) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during mlp_get_logits: expected " + std::to_string(want));
    ORCA_HIP_CHECK(hipMemcpyAsync(host, mlp->logits, n * sizeof(float), hipMemcpyDeviceToHost, mlp->ctx->stream));
    host_sync(mlp->ctx);
  });
}

int orca_hip_mlp_get_preds(orca_hip_mlp* mlp, int32_t* host, size_t n) {
  return guard([&] {
    checked(mlp);
    if (n != mlp->B) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during mlp_get_preds: expected " + std::to_string(mlp->B));
    ORCA_HIP_CHECK(hipMemcpyAsync(host, mlp->preds, n * sizeof(int32_t), hipMemcpyDeviceToHost, mlp->ctx->stream));
    host_sync(mlp->ctx);
  });
}

int orca_hip_mlp_get_activation(orca_hip_mlp* mlp, size_t layer, float* host, size_t n) {
  return guard([&] {
    checked(mlp);
    if (layer >= mlp->L) fail(ORCA_HIP_ERR_INTERNAL, "layer index out of range");
    size_t want = mlp->B * mlp->dims[layer + 1];
    if (n != want) fail(ORCA_HIP_ERR_SHAPE, "Shape mismatch during mlp_get_activation: expected " + std::to_string(want));
    const float* src = layer + 1 < mlp->L ? mlp->H[layer] : mlp->logits;
    ORCA_HIP_CHECK(hipMemcpyAsync(host, src, n * sizeof(float), hipMemcpyDeviceToHost, mlp->ctx->stream));
    host_sync(mlp->ctx);
  });
}

int orca_hip_mlp_get_step_count(const orca_hip_mlp* mlp, int64_t* t) {
  return guard([&] {
    if (!mlp || !t) fail(ORCA_HIP_ERR_INTERNAL, "null argument");
    *t = mlp->t;
  });
}

// The next step runs as step t + 1 (adamw.py:64 increments before use).
int orca_hip_mlp_set_step_count(orca_hip_mlp* mlp, int64_t t) {
  return guard([&] {
    checked(mlp);
    if (t < 0) fail(ORCA_HIP_ERR_INTERNAL, "step count must be >= 0");
    mlp->t = t;
  });
}

}  // extern "C"
