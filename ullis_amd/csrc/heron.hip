// One Heron train step on the device: UllisHeron::train_step_on
// (src/model.rs:2827-3025) with rosa_grad = stop_grad_bits, from the gathered
// embedding rows to the embedding-row gradient, as a single stream of kernel
// launches with no host synchronisation.
//
// Order of operations (and which weights each GEMM sees) follows the
// reference: per block forward LN0 (block 0) -> LN3 -> time-shift mix3 ->
// Q/K/V (sign bit-planes for the automaton) -> y = (2 idx - 1) e -> O (+x)
// -> LN2 -> mix -> key (ReLU^2) -> value (+x); LN_out; head + CE; LN_out
// backward; per block in reverse: CMix backward (value input gradient, value
// weight gradient, key input and weight gradients, x_k gradient), LN2
// backward (+= into g_x), ROSA O stop-grad backward (e, O weight and O bias
// gradients), LN0 backward at block 0.
// Tapes stay resident in HBM between the forward and the backward.
//
// Two streams. With the automaton's indices given and rosa_grad =
// stop_grad_bits, two parts of the step feed nothing else in it: the ROSA
// Q/K/V branch (LN3, its mixes and the Q/K/V GEMMs, whose sign bit-planes are
// an output only) and the O backward (O weight gradient and the e gradient;
// ROSA passes no gradient to x). They run on a second stream (default
// priority), ordered after their inputs by events, while the main stream
// carries the residual chain; the main stream waits for the second one before
// the end-of-step updates. Every buffer the second stream reads is final when
// its event is recorded (x_l, the per-boundary fp16 gradient gx16_b[l], the
// layer's amax slot), and it writes only buffers of its own.
//
// Parameter updates: each tensor is read only by its own layer's forward and
// backward, and the reference updates it after its last read, so no kernel
// later in the step reads an updated parameter. Every update is therefore
// deferred to the end of the step: the gradient partials of each tensor stay
// in their own buffers and four batched launches (vector steps, fp16 weight
// steps, packed latent / scale steps with the repack, bit transposes) apply
// them, with the same per-tensor arithmetic as updating each tensor at the
// reference's update call.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>
#include <vector>

#include "../../include/ullis_hip.h"
#include "common.hpp"
#include "context.hpp"
#include "ops.hpp"

using namespace ullis;

namespace {

struct Ln {
  uint16_t *w = nullptr, *b = nullptr;
  float *w_res = nullptr, *b_res = nullptr;
};

struct Packed {
  long out = 0, in = 0;
  uint32_t *bits = nullptr, *bits_t = nullptr;
  uint16_t *scale = nullptr, *bias = nullptr, *latent = nullptr;
  float *scale_res = nullptr, *bias_res = nullptr, *latent_res = nullptr;
};

struct Block {
  bool has_ln0 = false;
  Ln ln0, ln2, ln3;
  uint16_t *x_q = nullptr, *x_k = nullptr, *x_v = nullptr, *e = nullptr;
  float* e_res = nullptr;
  Packed q, k, v, o, key;
  uint16_t* cx_k = nullptr;
  float* cx_k_res = nullptr;
  uint16_t* value = nullptr;
  float* value_res = nullptr;
  // value^T [F][D], kept for the value input gradient of large products
  // (fp16_dx_wants_w_t; else null), rebuilt after every update
  uint16_t* value_t = nullptr;
};

}  // namespace

struct ullis_hip_heron {
  ullis_hip_ctx* ctx = nullptr;
  ullis_heron_dims dims{};
  long batch = 0, time = 0, rows = 0, D = 0, F = 0, V = 0, L = 0;
  std::vector<ullis_tensor_desc> descs;
  uint8_t* arena = nullptr;
  uint64_t arena_bytes = 0;
  Ln ln_out;
  Packed head;
  std::vector<Block> blocks;
  void* act = nullptr;  // one allocation for activations, tapes and scratch
  // activations / tapes
  float *resid = nullptr, *after_rosa = nullptr;
  // O products (bias + scale * y . S^T, before the residual add) of every
  // layer, computed at the step's start on the second stream
  float* o_pre = nullptr;
  uint16_t *ln16 = nullptr, *q16 = nullptr, *k16 = nullptr, *v16 = nullptr;
  uint16_t *y16 = nullptr, *ln2_16 = nullptr, *shifted16 = nullptr;
  uint8_t* idx_rm = nullptr;
  uint16_t *key16 = nullptr, *relu2_16 = nullptr, *gk16 = nullptr;
  uint16_t* value_t_all = nullptr;  // the blocks' value^T caches (Block::value_t)
  // fp16 copy of the (scaled) gradient at each layer boundary x_l, l = 0..L:
  // read by layer l's O backward and layer l-1's CMix backward
  uint16_t* gx16_b = nullptr;
  float* g_side = nullptr;       // O input-gradient scratch of the second stream's fallback path
  uint16_t* ln3_16 = nullptr;    // LN3 output scratch of the second stream's fallback path
  // second stream and its ordering events
  hipStream_t side = nullptr;
  std::vector<hipEvent_t> ev_fwd, ev_bwd, ev_o;
  hipEvent_t ev_join = nullptr, ev_head = nullptr, ev_start = nullptr;
  float *g_x = nullptr, *g_a = nullptr, *g_b = nullptr;
  float *slots = nullptr, *stats = nullptr;
  float* row_loss = nullptr;
  // this step's count of token ids >= vocab and labels >= vocab (other than
  // the ignore id); when non-zero every update launch of the step returns
  // without changing anything, as train_step_on refuses such a step before
  // any update (src/model.rs:2852-2861)
  uint32_t* invalid = nullptr;
  // per-row diagnostics the packed finishes write (CausalLoss): sign-bit
  // flips of every key / O / head row, the head rows' summed |latent step|,
  // and the head's scale gradient
  uint32_t *flips_key = nullptr, *flips_o = nullptr, *flips_head = nullptr;
  float *step_head = nullptr, *gscale_head = nullptr;
  void* diag_ws = nullptr;
  // gradient partials, one buffer per tensor, consumed by the end-of-step updates
  float *gp_value = nullptr, *gp_key = nullptr, *gp_o = nullptr, *gp_head = nullptr;
  float *pt_mix = nullptr, *pt_ln2 = nullptr, *pt_ob = nullptr, *pt_e = nullptr;
  float *pt_lnout = nullptr, *pt_ln0 = nullptr;
  int nb_col = 0, nb_ln = 0, nb_mix = 0;
  // batched update job tables (device memory) and their grid sizes; the LN0
  // job is the last vector job so that it can be left out when LN0 backward
  // took a path with another partial count (unaligned x_emb)
  void* job_mem = nullptr;
  const VecJob* vec_jobs = nullptr;
  const F16Job* f16_jobs = nullptr;
  const FinishJob* fin_jobs = nullptr;
  const TransJob* trans_jobs = nullptr;
  // The tables are cut into L + 2 segments: segment l holds layer l's jobs
  // (run on the second stream once its O backward is done), segment L the
  // LN_out and head jobs (on the second stream once LN_out's backward is
  // done), segment L + 1 the LN0 job (at the step's end); block0 values start
  // at 0 in every segment.
  struct JobRange {
    int j0 = 0, n = 0, blocks = 0;
  };
  struct UpdateSeg {
    JobRange vec, f16, fin, trans;
  };
  std::vector<UpdateSeg> seg;
  std::vector<const Packed*> trans_generic;  // bits_t rebuilt by the generic transpose
  // ROSA e of every layer (host array and a device copy) for the expand of all
  // layers' ROSA outputs in one launch
  std::vector<const uint16_t*> e_host;
  const uint16_t* const* e_dev = nullptr;
  uint32_t* qkv = nullptr;
  void* head_ws = nullptr;
  // live suffix automaton (ullis_hip_heron_step_sam), allocated on first use:
  // pinned host planes of one layer and indices of one layer, the device
  // indices of every layer, and the event the host waits on
  uint32_t* sam_planes_host = nullptr;
  uint8_t* sam_idx_host = nullptr;
  uint8_t* sam_idx_dev = nullptr;
  hipEvent_t ev_sam = nullptr;
  // T = 1 decode state (ullis_hip_heron_decode_*), one allocation
  struct Decode {
    long batch = 0;
    int parity = 0;  // which half of the previous-token buffers this token reads
    bool eager = false;  // no graph replay (ULLIS_HIP_DECODE_EAGER)
    void* mem = nullptr;
    // the previous token's LN3 / LN2 outputs per layer, [2][L][batch][D]:
    // a token reads half `parity` and writes the other
    float *rosa_prev = nullptr, *cmix_prev = nullptr;
    float *x = nullptr, *x2 = nullptr, *ln = nullptr;                            // [batch][D]
    float *q = nullptr, *k = nullptr, *v = nullptr;                              // [batch][D]
    uint16_t *q16 = nullptr, *k16 = nullptr, *v16 = nullptr, *y16 = nullptr, *sh16 = nullptr;
    uint16_t *hid16 = nullptr, *key16 = nullptr, *r2_16 = nullptr;  // [batch][D], [batch][F] x 2
    uint8_t *idx = nullptr, *idx_rm = nullptr;    // [batch][D]
    uint32_t* planes = nullptr;                   // [3][words]
    uint32_t* planes_host = nullptr;              // pinned
    uint8_t* idx_host = nullptr;                  // pinned
    // graphs of the step with the automaton's indices given, one per parity,
    // for the pointers in `key`
    struct Key {
      const void* p[6];
      long vocab;
      bool operator==(const Key& o) const {
        for (int i = 0; i < 6; ++i)
          if (p[i] != o.p[i]) return false;
        return vocab == o.vocab;
      }
    };
    hipGraphExec_t graph[2] = {nullptr, nullptr};
    Key graph_key[2] = {};
  } dec;
  int splits_o = 1, splits_key = 1, splits_value = 1;
  // kernel probe: events around every launch of one launch class
  int probe = 0;
  bool probe_events_only = false;  // ULLIS_HIP_PROBE_EVENTS: GEMMs timed by events too
  int probe_used = 0;
  std::vector<hipEvent_t> probe_events;
  // phase timing (ullis_hip_heron_phases): events on the main stream at the
  // boundaries of the reference's TrainStepProfile phases; phase_id[i] is the
  // phase of the segment that starts at event i (-1: a step's end)
  bool phase_on = false;
  int phase_n = 0;
  std::vector<hipEvent_t> phase_ev;
  std::vector<int> phase_id;
  unsigned long long* probe_stamps = nullptr;  // device [kStampTotal][2], lazily
  std::vector<long> probe_blocks;              // per probed launch: stamped blocks, 0 = events
  std::vector<long> probe_offset;              // per probed launch: first stamp slot
  long stamp_used = 0;                         // stamp slots taken since the probe was armed
  double wall_khz = 0.0;                       // device wall-clock rate (s_memrealtime)
  // step graph (ullis_hip_heron_set_graph): the launches of one step on both
  // streams, captured once and replayed while the step's arguments repeat
  struct StepArgs {
    const void* p[11];
    uint32_t ignore_id;
    float lr;
    long vocab;  // embedding rows of a step from token ids, else -1
    bool operator==(const StepArgs& o) const {
      for (int i = 0; i < 11; ++i)
        if (p[i] != o.p[i]) return false;
      return ignore_id == o.ignore_id && lr == o.lr && vocab == o.vocab;
    }
  };
  bool graph_on = false;
  hipGraphExec_t graph_exec = nullptr;
  StepArgs graph_args{};

  template <class T>
  T* tensor(const std::string& name) {
    const uint64_t off = ullis_heron_offset(descs.data(), descs.size(), name.c_str());
    if (off == UINT64_MAX) return nullptr;
    return reinterpret_cast<T*>(arena + off);
  }
};

namespace {

bool bind_ln(ullis_hip_heron* h, const std::string& p, Ln& l) {
  l.w = h->tensor<uint16_t>(p + ".weight");
  l.b = h->tensor<uint16_t>(p + ".bias");
  l.w_res = h->tensor<float>(p + ".weight.residual");
  l.b_res = h->tensor<float>(p + ".bias.residual");
  return l.w && l.b && l.w_res && l.b_res;
}

bool bind_packed(ullis_hip_heron* h, const std::string& p, long out, long in, bool bias,
                 bool transpose, Packed& k) {
  k.out = out;
  k.in = in;
  k.bits = h->tensor<uint32_t>(p + ".bits");
  k.bits_t = transpose ? h->tensor<uint32_t>(p + ".bits_t") : nullptr;
  k.scale = h->tensor<uint16_t>(p + ".scale");
  k.scale_res = h->tensor<float>(p + ".scale.residual");
  k.latent = h->tensor<uint16_t>(p + ".latent");
  k.latent_res = h->tensor<float>(p + ".latent.residual");
  if (bias) {
    k.bias = h->tensor<uint16_t>(p + ".bias");
    k.bias_res = h->tensor<float>(p + ".bias.residual");
  }
  return k.bits && (!transpose || k.bits_t) && k.scale && k.scale_res && k.latent &&
         k.latent_res && (!bias || (k.bias && k.bias_res));
}

#define STEP(expr, what)                              \
  do {                                                \
    if (int rc_ = c->hip((expr), (what))) return rc_; \
  } while (0)

constexpr int kProbeMax = 512;
constexpr int kPhaseMax = 2048;
// The reference's phase names (TrainStepProfile, src/model.rs:2864-2994).
enum Phase : int {
  kPhEmbed = 0, kPhFwdLn, kPhFwdRosa, kPhFwdCmix, kPhHead, kPhBwdLn, kPhBwdCmix, kPhBwdRosa,
  kPhEmbedSgd, kPhEnd = -1
};
static_assert(kPhEmbedSgd + 1 == ULLIS_HIP_PHASE_COUNT, "phase names");
// Marks the start of phase k on stream `st` when phase timing is on.
#define PHASE_AT(st, k)                                                          \
  do {                                                                           \
    if (h->phase_on && h->phase_n < kPhaseMax) {                                 \
      STEP(hipEventRecord(h->phase_ev[h->phase_n], (st)), "phase event");       \
      h->phase_id[h->phase_n++] = (k);                                           \
    }                                                                            \
  } while (0)
// (start, end) slots for every workgroup of the stamped launches of one probe
// pass; a launch that no longer fits is timed by events instead
constexpr long kStampTotal = 1L << 22;

__global__ void probe_stamps_clear_kernel(unsigned long long* st, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) st[i] = 0ull;
}

// When `id` is the probed launch class, the kernel that `expr` launches
// records its execution interval (LaunchProbe: device wall-clock stamps for
// the streamed-LDS GEMMs, kernel-timestamp events for other kernels). `expr`
// must launch exactly one kernel.
#define PROBED(id, expr, what)                                                     \
  do {                                                                             \
    const bool on_ = h->probe == (id) && h->probe_used < kProbeMax;                \
    LaunchProbe lp_;                                                               \
    if (on_) {                                                                     \
      lp_.start = h->probe_events[2 * h->probe_used];                              \
      lp_.stop = h->probe_events[2 * h->probe_used + 1];                           \
      lp_.stamps = h->probe_events_only ? nullptr : h->probe_stamps + 2 * h->stamp_used; \
      lp_.stamp_cap = kStampTotal - h->stamp_used;                                 \
      t_launch_probe = &lp_;                                                       \
    }                                                                              \
    const int rc_ = c->hip((expr), (what));                                        \
    const bool consumed_ = t_launch_probe == nullptr;                              \
    t_launch_probe = nullptr;                                                      \
    if (rc_) return rc_;                                                           \
    if (on_) {                                                                     \
      if (!consumed_) return c->fail(ULLIS_HIP_ERR_RUNTIME, "probe: no kernel launched"); \
      h->probe_blocks[h->probe_used] = lp_.used_stamps ? lp_.blocks : 0;           \
      h->probe_offset[h->probe_used] = h->stamp_used;                              \
      if (lp_.used_stamps) h->stamp_used += lp_.blocks;                            \
      ++h->probe_used;                                                             \
    }                                                                              \
  } while (0)

// Brackets a multi-kernel operation with events when `id` is the probed class.
#define PROBED_SPAN(id, expr, what)                                                \
  do {                                                                             \
    const bool on_ = h->probe == (id) && h->probe_used < kProbeMax;                \
    if (on_) STEP(hipEventRecord(h->probe_events[2 * h->probe_used], s), "probe"); \
    STEP(expr, what);                                                              \
    if (on_) {                                                                     \
      STEP(hipEventRecord(h->probe_events[2 * h->probe_used + 1], s), "probe");    \
      h->probe_blocks[h->probe_used] = 0;                                          \
      ++h->probe_used;                                                             \
    }                                                                              \
  } while (0)

struct HeronSegStart {
  int v, f, p, t;
};

// Job tables of the end-of-step updates (every pointer in them is fixed for
// the life of the trainer), uploaded once.
int build_update_jobs(ullis_hip_heron* h) {
  ullis_hip_ctx* c = h->ctx;
  const long R = h->rows, D = h->D, F = h->F, V = h->V, L = h->L;
  const float ste = (float)(h->time - 1);  // binaryconnect_ste_scale(time - 1), src/model.rs:554-556
  std::vector<VecJob> vj;
  std::vector<F16Job> fj;
  std::vector<FinishJob> pj;
  std::vector<TransJob> tj;
  int vb = 0, fb = 0, pb = 0, tb = 0;  // blocks of the open segment
  bool vec_ok = true;
  auto open_seg = [&] {
    HeronSegStart st{(int)vj.size(), (int)fj.size(), (int)pj.size(), (int)tj.size()};
    vb = fb = pb = tb = 0;
    return st;
  };
  auto close_seg = [&](const HeronSegStart& st) {
    ullis_hip_heron::UpdateSeg g;
    g.vec = {st.v, (int)vj.size() - st.v, vb};
    g.f16 = {st.f, (int)fj.size() - st.f, fb};
    g.fin = {st.p, (int)pj.size() - st.p, pb};
    g.trans = {st.t, (int)tj.size() - st.t, tb};
    h->seg.push_back(g);
  };
  auto vec2 = [&](const float* part, int nblk, long ch, bool two, VecTarget a, VecTarget b) {
    VecJob j{part, nblk, two ? 2 * ch : ch, ch, a, two ? b : a, vb};
    vb += vec_job_blocks(j.ncols);
    vj.push_back(j);
  };
  auto sgd = [](uint16_t* v, float* r, float mult, const float* mul) {
    return VecTarget{nullptr, v, r, mult, mul};
  };
  auto ln = [&](const Ln& n, const float* part, int nblk) {
    vec2(part, nblk, D, true, sgd(n.w, n.w_res, 1.0f, nullptr), sgd(n.b, n.b_res, 1.0f, nullptr));
  };
  // packed latent / scale steps with the repack (rows of in % 32 == 0
  // weights), then the bit transpose
  auto packed = [&](const Packed& k, long row0, long rows, const float* part, int splits,
                    const float* amax, const float* extra_mul, uint32_t* row_flips,
                    float* row_step = nullptr, float* g_scale = nullptr) {
    PackedFinish f;
    f.part = part;
    f.splits = splits;
    f.out = rows;
    f.in = k.in;
    f.scale = k.scale + row0;
    f.bits_old = k.bits + row0 * k.in / 32;
    f.amax = amax;
    f.extra_mul = extra_mul;
    f.ste = ste;
    f.lr = 0.0f;
    f.latent = k.latent + row0 * k.in;
    f.latent_res = k.latent_res + row0 * k.in;
    f.g_scale = g_scale;
    f.g_w = nullptr;
    f.scale_upd = k.scale + row0;
    f.scale_res = k.scale_res + row0;
    f.bits_new = k.bits + row0 * k.in / 32;
    f.row_flips = row_flips;
    f.row_step = row_step;
    vec_ok = vec_ok && packed_finish_wave_ok(f);
    pj.push_back(FinishJob{f, pb});
    pb += finish_job_blocks(rows);
  };
  auto rebuild = [&](const Packed& k) {
    if (!k.bits_t) return;
    if (k.out % 32 == 0 && k.in % 32 == 0) {
      tj.push_back(TransJob{k.bits, k.out, k.in, k.bits_t, tb});
      tb += (int)cdiv((k.out / 32) * (k.in / 32), 8);
    } else {
      h->trans_generic.push_back(&k);
    }
  };

  for (long l = 0; l < L; ++l) {
    const HeronSegStart st = open_seg();
    Block& b = h->blocks[l];
    const long pc = (long)h->nb_col * D;
    vec2(h->pt_mix + l * h->nb_mix * D, h->nb_mix, D, false, sgd(b.cx_k, b.cx_k_res, 1.0f, nullptr),
         {});
    ln(b.ln2, h->pt_ln2 + l * 2L * h->nb_ln * D, h->nb_ln);
    vec2(h->pt_ob + l * pc, h->nb_col, D, false, sgd(b.o.bias, b.o.bias_res, 1.0f, nullptr), {});
    vec2(h->pt_e + l * pc, h->nb_col, D, false, sgd(b.e, b.e_res, 1.0f, nullptr), {});
    const long nv = D * F;
    const float* gpv = h->gp_value + l * h->splits_value * nv;
    vec_ok = vec_ok && fp16_finish_vec_ok(gpv, nv, b.value, b.value_res, nullptr);
    fj.push_back(F16Job{gpv, h->splits_value, nv, h->slots + l + 1, b.value, b.value_res, fb});
    fb += f16_job_blocks(nv);
    packed(b.key, 0, F, h->gp_key + l * h->splits_key * F * D, h->splits_key, h->slots + l + 1,
           nullptr, h->flips_key + l * F);
    packed(b.o, 0, D, h->gp_o + l * h->splits_o * D * D, h->splits_o, h->slots + l, nullptr,
           h->flips_o + l * D);
    rebuild(b.key);
    rebuild(b.o);
    close_seg(st);
  }
  const HeronSegStart tail = open_seg();
  ln(h->ln_out, h->pt_lnout, h->nb_ln);
  // head bias: g_bias = gscale * column sums, step at 8 lr (src/model.rs:3118-3130)
  vec2(head_ce_bias_partials(h->head_ws, R, D, V), (int)cdiv(R, 32), V, false,
       sgd(h->head.bias, h->head.bias_res, kHeadBiasLrMult, h->stats + 2), {});
  {
    const long vc = head_ce_chunk_cols(V, D);
    const int sp = head_ce_splits(R, D, V);
    for (long c0 = 0, ci = 0; c0 < V; c0 += vc, ++ci)
      packed(h->head, c0, V - c0 < vc ? V - c0 : vc, h->gp_head + ci * sp * vc * D, sp, nullptr,
             h->stats + 2, h->flips_head + c0, h->step_head + c0, h->gscale_head + c0);
  }
  rebuild(h->head);
  close_seg(tail);
  const HeronSegStart last = open_seg();
  if (h->blocks[0].has_ln0) ln(h->blocks[0].ln0, h->pt_ln0, h->nb_ln);
  close_seg(last);
  if (!vec_ok)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron update tensors are not 16-byte aligned");

  size_t bytes = 0;
  auto add = [&](size_t b) { bytes += Carver::bytes_for(b); };
  add(sizeof(VecJob) * vj.size());
  add(sizeof(F16Job) * fj.size());
  add(sizeof(FinishJob) * pj.size());
  add(sizeof(TransJob) * tj.size());
  for (const Block& b : h->blocks) h->e_host.push_back(b.e);
  add(sizeof(const uint16_t*) * h->e_host.size());
  if (int rc = c->hip(hipMalloc(&h->job_mem, bytes), "heron update job tables")) return rc;
  Carver cv(h->job_mem);
  auto up = [&](auto& v, auto*& dst, int& n) -> int {
    using J = typename std::remove_reference_t<decltype(v)>::value_type;
    J* d = cv.take<J>(v.size());
    dst = d;
    n = (int)v.size();
    if (v.empty()) return 0;
    return c->hip(hipMemcpy(d, v.data(), sizeof(J) * v.size(), hipMemcpyHostToDevice),
                  "heron update job upload");
  };
  int n = 0;
  if (int rc = up(vj, h->vec_jobs, n)) return rc;
  if (int rc = up(fj, h->f16_jobs, n)) return rc;
  if (int rc = up(pj, h->fin_jobs, n)) return rc;
  if (int rc = up(tj, h->trans_jobs, n)) return rc;
  if (int rc = up(h->e_host, h->e_dev, n)) return rc;
  return 0;
}

// The update launches of one segment.
int run_update_seg(ullis_hip_heron* h, hipStream_t s, int l, float lr) {
  ullis_hip_ctx* c = h->ctx;
  const ullis_hip_heron::UpdateSeg& g = h->seg[l];
  // vector steps (LN gamma / beta, x_k, O bias, e, head bias at 8 lr)
  STEP(run_vec_jobs(s, h->vec_jobs + g.vec.j0, g.vec.n, g.vec.blocks, lr, h->invalid),
       "vector steps");
  STEP(run_f16_jobs(s, h->f16_jobs + g.f16.j0, g.f16.n, g.f16.blocks, lr, h->invalid),
       "value steps");
  STEP(run_finish_jobs(s, h->fin_jobs + g.fin.j0, g.fin.n, g.fin.blocks, lr, h->invalid),
       "latent / scale steps");
  STEP(run_trans_jobs(s, h->trans_jobs + g.trans.j0, g.trans.n, g.trans.blocks, h->invalid),
       "bits_t");
  // the value weight's transpose for the next step's input gradient (a
  // refused step changed nothing, so transposing again is harmless)
  if (l < (int)h->L && h->blocks[l].value_t)
    STEP(transpose_u16(s, h->blocks[l].value, h->D, h->F, h->blocks[l].value_t), "value^T");
  return 0;
}

}  // namespace

extern "C" {

int ullis_hip_heron_create(ullis_hip_ctx* c, const ullis_heron_dims* dims, size_t batch,
                           size_t time, ullis_hip_heron** out) {
  if (!c || !dims || !out) return ULLIS_HIP_ERR_INVALID;
  *out = nullptr;
  if (dims->d_model == 0 || dims->n_layers == 0 || dims->dim_ffn == 0 || dims->vocab == 0 ||
      batch == 0 || time < 2)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron dims must be non-zero and time >= 2");
  if (dims->d_model % 32 != 0)
    return c->fail(ULLIS_HIP_ERR_INVALID, "d_model must be a multiple of 32 (sign bit-planes)");
  if ((double)batch * time * dims->dim_ffn > (double)INT32_MAX ||
      (double)dims->vocab * dims->d_model > (double)INT32_MAX)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron shape exceeds int32 extents");
  auto* h = new ullis_hip_heron();
  h->ctx = c;
  h->dims = *dims;
  h->batch = (long)batch;
  h->time = (long)time;
  h->rows = (long)(batch * time);
  h->D = dims->d_model;
  h->F = dims->dim_ffn;
  h->V = dims->vocab;
  h->L = dims->n_layers;
  const size_t n = ullis_heron_layout(dims, nullptr, 0, &h->arena_bytes);
  h->descs.resize(n);
  ullis_heron_layout(dims, h->descs.data(), n, &h->arena_bytes);
  if (hipMalloc(&h->arena, h->arena_bytes) != hipSuccess) {
    delete h;
    return c->fail(ULLIS_HIP_ERR_NOMEM, "heron arena allocation failed");
  }
  (void)hipMemsetAsync(h->arena, 0, h->arena_bytes, c->stream);

  bool ok = bind_ln(h, "ln_out", h->ln_out) && bind_packed(h, "head", h->V, h->D, true, true, h->head);
  h->blocks.resize(h->L);
  for (long l = 0; l < h->L && ok; ++l) {
    Block& b = h->blocks[l];
    const std::string p = "blocks." + std::to_string(l);
    b.has_ln0 = l == 0;
    if (b.has_ln0) ok = ok && bind_ln(h, p + ".ln0", b.ln0);
    ok = ok && bind_ln(h, p + ".ln2", b.ln2) && bind_ln(h, p + ".ln3", b.ln3);
    b.x_q = h->tensor<uint16_t>(p + ".rosa.x_q");
    b.x_k = h->tensor<uint16_t>(p + ".rosa.x_k");
    b.x_v = h->tensor<uint16_t>(p + ".rosa.x_v");
    b.e = h->tensor<uint16_t>(p + ".rosa.e");
    b.e_res = h->tensor<float>(p + ".rosa.e.residual");
    b.cx_k = h->tensor<uint16_t>(p + ".ffn.x_k");
    b.cx_k_res = h->tensor<float>(p + ".ffn.x_k.residual");
    b.value = h->tensor<uint16_t>(p + ".ffn.value");
    b.value_res = h->tensor<float>(p + ".ffn.value.residual");
    ok = ok && b.x_q && b.x_k && b.x_v && b.e && b.e_res && b.cx_k && b.cx_k_res && b.value &&
         b.value_res;
    ok = ok && bind_packed(h, p + ".rosa.q", h->D, h->D, true, false, b.q) &&
         bind_packed(h, p + ".rosa.k", h->D, h->D, true, false, b.k) &&
         bind_packed(h, p + ".rosa.v", h->D, h->D, true, false, b.v) &&
         bind_packed(h, p + ".rosa.o", h->D, h->D, true, true, b.o) &&
         bind_packed(h, p + ".ffn.key", h->F, h->D, false, true, b.key);
  }
  if (!ok) {
    (void)hipFree(h->arena);
    delete h;
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron arena layout is missing a tensor");
  }

  const long R = h->rows, D = h->D, F = h->F, L = h->L, V = h->V;
  const long nd = R * D, nf = R * F;
  const long words = cdiv(nd, 32);
  h->splits_o = pair_dw_splits(D, D, R);
  h->splits_key = pair_dw_splits(F, D, R);
  h->splits_value = pair_dw_splits(D, F, R);
  h->nb_col = (int)column_partial_blocks(R);
  h->nb_ln = layer_norm_backward_nblk(R, D);
  h->nb_mix = layer_norm_mix_backward_mix_nblk(R, D);
  const long nb_ln0 = layer_norm_backward_blocks(R);  // any LN backward path fits
  const long head_vc = head_ce_chunk_cols(V, D);
  const long head_sp = head_ce_splits(R, D, V);
  const long head_chunks = cdiv(V, head_vc);
  const long gp_value = (long)h->splits_value * D * F, gp_key = (long)h->splits_key * F * D;
  const long gp_o = (long)h->splits_o * D * D, gp_head = head_chunks * head_sp * head_vc * D;
  const long pt_col = (long)h->nb_col * D, pt_ln = 2L * h->nb_ln * D;
  const long pt_mix = (long)h->nb_mix * D;
  const size_t head_ws = head_ce_workspace_bytes(R, D, V);
  const long value_t_elems = fp16_dx_wants_w_t(R, F, D) ? F * D * L : 0;

  // one carving sequence, run once to size the allocation and once to place the buffers
  auto carve = [&](auto& cv) {
    h->resid = cv.template take<float>(nd * (L + 1));
    h->after_rosa = cv.template take<float>(nd * L);
    h->o_pre = cv.template take<float>(nd * L);
    h->ln16 = cv.template take<uint16_t>(nd);
    h->q16 = cv.template take<uint16_t>(nd);
    h->k16 = cv.template take<uint16_t>(nd);
    h->v16 = cv.template take<uint16_t>(nd);
    h->y16 = cv.template take<uint16_t>(nd * L);
    h->ln2_16 = cv.template take<uint16_t>(nd * L);
    h->shifted16 = cv.template take<uint16_t>(nd * L);
    h->idx_rm = cv.template take<uint8_t>(nd * L);
    h->key16 = cv.template take<uint16_t>(nf * L);
    h->relu2_16 = cv.template take<uint16_t>(nf * L);
    h->gk16 = cv.template take<uint16_t>(nf);
    // (a zero-length take would still return a pointer into the next buffer)
    h->value_t_all = value_t_elems ? cv.template take<uint16_t>(value_t_elems) : nullptr;
    h->gx16_b = cv.template take<uint16_t>(nd * (L + 1));
    h->g_side = cv.template take<float>(nd);
    h->ln3_16 = cv.template take<uint16_t>(nd);
    h->g_x = cv.template take<float>(nd);
    h->g_a = cv.template take<float>(nd);
    h->g_b = cv.template take<float>(nd);
    h->gp_value = cv.template take<float>(gp_value * L);
    h->gp_key = cv.template take<float>(gp_key * L);
    h->gp_o = cv.template take<float>(gp_o * L);
    h->gp_head = cv.template take<float>(gp_head);
    h->pt_mix = cv.template take<float>(pt_mix * L);
    h->pt_ob = cv.template take<float>(pt_col * L);
    h->pt_e = cv.template take<float>(pt_col * L);
    h->pt_ln2 = cv.template take<float>(pt_ln * L);
    h->pt_lnout = cv.template take<float>(pt_ln);
    h->pt_ln0 = cv.template take<float>(2 * nb_ln0 * D);
    h->slots = cv.template take<float>(L + 2);
    h->stats = cv.template take<float>(4);
    h->row_loss = cv.template take<float>(R);
    h->qkv = cv.template take<uint32_t>(words * 3 * L);
    h->head_ws = cv.template take<char>(head_ws);
    h->invalid = cv.template take<uint32_t>(1);
    h->flips_key = cv.template take<uint32_t>(F * L);
    h->flips_o = cv.template take<uint32_t>(D * L);
    h->flips_head = cv.template take<uint32_t>(V);
    h->step_head = cv.template take<float>(V);
    h->gscale_head = cv.template take<float>(V);
    h->diag_ws = cv.template take<char>(diag_workspace_bytes(V));
  };
  CarveSizer sizer;
  carve(sizer);
  if (hipMalloc(&h->act, sizer.used) != hipSuccess) {
    (void)hipFree(h->arena);
    delete h;
    return c->fail(ULLIS_HIP_ERR_NOMEM, "heron activation allocation of " +
                                            std::to_string(sizer.used) + " bytes failed");
  }
  Carver cv(h->act);
  carve(cv);
  if (h->value_t_all)
    for (long l = 0; l < L; ++l) h->blocks[l].value_t = h->value_t_all + l * F * D;
  if (int rc = build_update_jobs(h)) {
    ullis_hip_heron_destroy(h);
    return rc;
  }
  {
    bool ok2 = hipStreamCreateWithFlags(&h->side, hipStreamNonBlocking) == hipSuccess;
    h->ev_fwd.assign(L, nullptr);
    h->ev_bwd.assign(L, nullptr);
    h->ev_o.assign(L, nullptr);
    for (auto* v : {&h->ev_fwd, &h->ev_bwd, &h->ev_o})
      for (auto& e : *v) ok2 = ok2 && hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess;
    ok2 = ok2 && hipEventCreateWithFlags(&h->ev_join, hipEventDisableTiming) == hipSuccess;
    ok2 = ok2 && hipEventCreateWithFlags(&h->ev_start, hipEventDisableTiming) == hipSuccess;
    ok2 = ok2 && hipEventCreateWithFlags(&h->ev_head, hipEventDisableTiming) == hipSuccess;
    if (!ok2) {
      ullis_hip_heron_destroy(h);
      return c->fail(ULLIS_HIP_ERR_RUNTIME, "heron stream / event creation failed");
    }
  }
  h->probe_blocks.assign(kProbeMax, 0);
  h->probe_offset.assign(kProbeMax, 0);
  {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess ||
        khz <= 0) {
      ullis_hip_heron_destroy(h);
      return c->fail(ULLIS_HIP_ERR_RUNTIME, "device wall-clock rate unavailable");
    }
    h->wall_khz = (double)khz;
  }
  h->probe_events.resize(2 * kProbeMax);
  for (auto& e : h->probe_events) {
    if (hipEventCreate(&e) != hipSuccess) {
      e = nullptr;
      ullis_hip_heron_destroy(h);
      return c->fail(ULLIS_HIP_ERR_RUNTIME, "probe event creation failed");
    }
  }
  if (int rc = c->hip(hipStreamSynchronize(c->stream), "heron create")) {
    ullis_hip_heron_destroy(h);
    return rc;
  }
  *out = h;
  return 0;
}

void ullis_hip_heron_destroy(ullis_hip_heron* h) {
  if (!h) return;
  if (h->ctx) (void)hipStreamSynchronize(h->ctx->stream);
  for (auto& e : h->probe_events) (void)hipEventDestroy(e);
  for (auto& e : h->phase_ev) (void)hipEventDestroy(e);
  if (h->side) (void)hipStreamSynchronize(h->side);
  for (auto* v : {&h->ev_fwd, &h->ev_bwd, &h->ev_o})
    for (auto& e : *v)
      if (e) (void)hipEventDestroy(e);
  if (h->ev_join) (void)hipEventDestroy(h->ev_join);
  if (h->ev_start) (void)hipEventDestroy(h->ev_start);
  if (h->ev_head) (void)hipEventDestroy(h->ev_head);
  if (h->side) (void)hipStreamDestroy(h->side);
  if (h->arena) (void)hipFree(h->arena);
  if (h->act) (void)hipFree(h->act);
  if (h->job_mem) (void)hipFree(h->job_mem);
  if (h->probe_stamps) (void)hipFree(h->probe_stamps);
  if (h->sam_planes_host) (void)hipHostFree(h->sam_planes_host);
  if (h->sam_idx_host) (void)hipHostFree(h->sam_idx_host);
  if (h->sam_idx_dev) (void)hipFree(h->sam_idx_dev);
  if (h->ev_sam) (void)hipEventDestroy(h->ev_sam);
  for (auto& g : h->dec.graph)
    if (g) (void)hipGraphExecDestroy(g);
  if (h->dec.mem) (void)hipFree(h->dec.mem);
  if (h->dec.planes_host) (void)hipHostFree(h->dec.planes_host);
  if (h->dec.idx_host) (void)hipHostFree(h->dec.idx_host);
  if (h->graph_exec) (void)hipGraphExecDestroy(h->graph_exec);
  delete h;
}

int ullis_hip_heron_arena(ullis_hip_heron* h, void** device_ptr, uint64_t* bytes) {
  if (!h || !device_ptr || !bytes) return ULLIS_HIP_ERR_INVALID;
  *device_ptr = h->arena;
  *bytes = h->arena_bytes;
  return 0;
}

int ullis_hip_heron_probe(ullis_hip_heron* h, int probe_id) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  const bool events_only = (probe_id & ULLIS_HIP_PROBE_EVENTS) != 0;
  probe_id &= ~ULLIS_HIP_PROBE_EVENTS;
  if (probe_id < 0 || probe_id >= ULLIS_HIP_PROBE_COUNT) return ULLIS_HIP_ERR_INVALID;
  h->probe = probe_id;
  h->probe_events_only = events_only;
  h->probe_used = 0;
  h->stamp_used = 0;
  if (probe_id != ULLIS_HIP_PROBE_NONE) {
    ullis_hip_ctx* c = h->ctx;
    const long n = 2 * kStampTotal;
    if (!h->probe_stamps)
      STEP(hipMalloc(&h->probe_stamps, sizeof(unsigned long long) * n), "probe stamps alloc");
    launch(probe_stamps_clear_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, c->stream,
           h->probe_stamps, n);
    STEP(hipGetLastError(), "probe stamps clear");
  }
  return 0;
}

int ullis_hip_heron_phases(ullis_hip_heron* h, int enable) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  if (enable && h->phase_ev.empty()) {
    h->phase_ev.assign(kPhaseMax, nullptr);
    h->phase_id.assign(kPhaseMax, kPhEnd);
    for (auto& e : h->phase_ev)
      if (hipEventCreate(&e) != hipSuccess) {
        (void)hipGetLastError();
        return c->fail(ULLIS_HIP_ERR_RUNTIME, "phase event creation failed");
      }
  }
  h->phase_on = enable != 0;
  h->phase_n = 0;
  return 0;
}

int ullis_hip_heron_phases_read(ullis_hip_heron* h, float* ms, int* steps) {
  if (!h || !ms || !steps) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  STEP(hipStreamSynchronize(c->stream), "phases sync");
  STEP(hipStreamSynchronize(h->side), "phases sync");
  if (h->phase_n >= kPhaseMax)
    return c->fail(ULLIS_HIP_ERR_INVALID, "phase event capacity exceeded: read after fewer steps");
  double sum[ULLIS_HIP_PHASE_COUNT] = {};
  int n = 0;
  for (int i = 0; i + 1 < h->phase_n; ++i) {
    if (h->phase_id[i] == kPhEnd) continue;
    float t = 0.0f;
    STEP(hipEventElapsedTime(&t, h->phase_ev[i], h->phase_ev[i + 1]), "phase elapsed");
    sum[h->phase_id[i]] += t;
  }
  for (int i = 0; i < h->phase_n; ++i) n += h->phase_id[i] == kPhEnd ? 1 : 0;
  for (int k = 0; k < ULLIS_HIP_PHASE_COUNT; ++k) ms[k] = (float)sum[k];
  *steps = n;
  return 0;
}

int ullis_hip_heron_probe_read(ullis_hip_heron* h, float* total_ms, int* launches) {
  if (!h || !total_ms || !launches) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  STEP(hipStreamSynchronize(c->stream), "probe sync");
  STEP(hipStreamSynchronize(h->side), "probe sync");
  std::vector<unsigned long long> st;
  double sum = 0.0;
  for (int i = 0; i < h->probe_used; ++i) {
    if (const long nb = h->probe_blocks[i]) {
      st.resize(2 * (size_t)nb);
      STEP(hipMemcpy(st.data(), h->probe_stamps + 2 * h->probe_offset[i],
                     sizeof(unsigned long long) * st.size(), hipMemcpyDeviceToHost),
           "probe stamps");
      unsigned long long t0 = ~0ull, t1 = 0;
      for (long b = 0; b < nb; ++b) {
        if (st[2 * b] == 0 || st[2 * b + 1] < st[2 * b])
          return c->fail(ULLIS_HIP_ERR_RUNTIME, "probe stamps unset");
        t0 = std::min(t0, st[2 * b]);
        t1 = std::max(t1, st[2 * b + 1]);
      }
      sum += (double)(t1 - t0) / h->wall_khz;
      continue;
    }
    float ms = 0.0f;
    STEP(hipEventSynchronize(h->probe_events[2 * i + 1]), "probe sync");
    STEP(hipEventElapsedTime(&ms, h->probe_events[2 * i], h->probe_events[2 * i + 1]),
         "probe elapsed");
    sum += ms;
  }
  *total_ms = (float)sum;
  *launches = h->probe_used;
  h->probe_used = 0;
  h->stamp_used = 0;
  return 0;
}

int ullis_hip_heron_refresh_derived(ullis_hip_heron* h) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  hipStream_t s = c->stream;
  STEP(transpose_bits(s, h->head.bits, h->head.out, h->head.in, h->head.bits_t), "head bits_t");
  for (auto& b : h->blocks) {
    STEP(transpose_bits(s, b.o.bits, b.o.out, b.o.in, b.o.bits_t), "o bits_t");
    STEP(transpose_bits(s, b.key.bits, b.key.out, b.key.in, b.key.bits_t), "key bits_t");
    if (b.value_t) STEP(transpose_u16(s, b.value, h->D, h->F, b.value_t), "value^T");
  }
  return 0;
}

}  // extern "C"

namespace {

// The embedding table a step from token ids updates (src/model.rs:2986-2993).
struct EmbedArgs {
  uint16_t* table;
  float* residual;
  long vocab;
  const uint32_t* tokens;
};

// Every launch of one train step, on the context stream and the second
// stream (arguments checked by ullis_hip_heron_step). With emb, the
// embedding scatter-SGD of g_emb runs as soon as g_emb is complete, beside
// the second stream's last updates.
// The suffix automaton of a step driven live, layer by layer, by the
// caller's callback (ullis_hip_heron_step_sam).
struct SamHandoff {
  ullis_hip_sam_fn fn;
  void* user;
};

int step_launches(ullis_hip_heron* h, const float* x_emb, const uint32_t* labels,
                  uint32_t ignore_id, float lr, const uint8_t* rosa_idx, float* g_emb,
                  float* row_loss, float* stats4, uint32_t* qkv_bits, uint32_t* invalid_out,
                  const EmbedArgs* emb = nullptr, const SamHandoff* live = nullptr) {
  ullis_hip_ctx* c = h->ctx;
  hipStream_t s = c->stream;
  const long R = h->rows, D = h->D, F = h->F, L = h->L, T = h->time, B = h->batch;
  const long nd = R * D, nf = R * F;
  const long words = cdiv(nd, 32);
  const float ste = (float)(T - 1);  // binaryconnect_ste_scale(time - 1), src/model.rs:554-556
  float* rl = row_loss ? row_loss : h->row_loss;
  uint32_t* qkv = qkv_bits ? qkv_bits : h->qkv;
  int nb = 0;
  bool ln0_now = false;

  PHASE_AT(s, kPhFwdRosa);
  STEP(fill_f32(s, h->slots, L + 2, 0.0f), "clear amax slots");
  // a step from token ids has cleared the counter before its gather
  if (!emb) STEP(fill_f32(s, reinterpret_cast<float*>(h->invalid), 1, 0.0f), "clear invalid");
  // y = (2 idx - 1) e (e is not updated before the step's end): layer 0's
  // here, the other layers' on the second stream after layer 0's O product
  // (with a live automaton, each layer's once its indices are back)
  if (!live)
    STEP(rosa_expand_layers(s, rosa_idx, h->e_host.data(), h->e_dev, 1, B, T, D, h->y16,
                            h->idx_rm),
         "rosa y");
  // The O products of every layer (src/model.rs:1428) read only y and the O
  // weights, all final here (updates run at the step's end): the second
  // stream computes them ahead of their layers, and each layer's LN2 adds its
  // residual x_l, so the residual chain no longer waits for an O GEMM per
  // layer. Layer 0's runs now; layer l + 1's is queued on the second stream
  // once x_l is complete, ahead of layer l's Q/K/V branch, which paces the
  // second stream's work with the layers instead of front-loading it.
  auto o_forward = [&](long l) -> int {
    const Block& b = h->blocks[l];
    PackedFwdOut o;
    o.y32 = h->o_pre + l * nd;
    STEP(packed_forward(h->side, h->y16 + l * nd, kF16, R, D, D, b.o.bits, b.o.scale, b.o.bias, o),
         "o");
    STEP(hipEventRecord(h->ev_o[l], h->side), "event");
    return 0;
  };
  STEP(hipEventRecord(h->ev_start, s), "event");
  STEP(hipStreamWaitEvent(h->side, h->ev_start, 0), "event wait");
  if (!live) {
    if (int rc = o_forward(0)) return rc;
    if (L > 1)
      STEP(rosa_expand_layers(h->side, rosa_idx + nd, h->e_host.data() + 1, h->e_dev + 1, L - 1,
                              B, T, D, h->y16 + nd, h->idx_rm + nd),
           "rosa y");
  }

  // ------------------------------------------------------------- forward
  for (long l = 0; l < L; ++l) {
    Block& b = h->blocks[l];
    float* x_l = h->resid + l * nd;
    if (b.has_ln0) {
      PHASE_AT(s, kPhFwdLn);
      STEP(layer_norm_forward(s, x_emb, R, D, b.ln0.w, b.ln0.b, x_l, nullptr), "ln0");
    } else if (l == 0) {
      STEP(copy_device(s, x_l, x_emb, (long)sizeof(float) * nd), "copy x");
    }
    // ROSA block (src/model.rs:1354-1440). With the automaton's indices
    // given, the Q/K/V branch runs on the second stream once x_l is
    // complete; with a live automaton it is on the residual chain: Q/K/V,
    // their sign bit-planes to the host, the caller's automaton, the indices
    // back, y = (2 idx - 1) e and the O product (src/metal.rs:1411-1511).
    hipStream_t qs = live ? s : h->side;
    PHASE_AT(s, kPhFwdRosa);
    if (!live) {
      STEP(hipEventRecord(h->ev_fwd[l], s), "event");
      STEP(hipStreamWaitEvent(h->side, h->ev_fwd[l], 0), "event wait");
      if (l + 1 < L)
        if (int rc = o_forward(l + 1)) return rc;
    }
    STEP(layer_norm_mix_forward(qs, x_l, R, T, D, b.ln3.w, b.ln3.b, h->ln3_16, false, b.x_q,
                                h->q16, b.x_k, h->k16, b.x_v, h->v16),
         "ln3 + mix3");
    {
      const uint16_t* const xin[3] = {h->q16, h->k16, h->v16};
      const uint32_t* const wb[3] = {b.q.bits, b.k.bits, b.v.bits};
      const uint16_t* const sc[3] = {b.q.scale, b.k.scale, b.v.scale};
      const uint16_t* const bi[3] = {b.q.bias, b.k.bias, b.v.bias};
      uint32_t* const planes[3] = {qkv + (l * 3 + 0) * words, qkv + (l * 3 + 1) * words,
                                   qkv + (l * 3 + 2) * words};
      STEP(packed_forward_bits3(qs, xin, R, D, D, wb, sc, bi, planes), "qkv");
    }
    if (live) {
      // planes out (pinned host memory), the callback, indices back
      STEP(hipMemcpyAsync(h->sam_planes_host, qkv + l * 3 * words, sizeof(uint32_t) * 3 * words,
                          hipMemcpyDeviceToHost, s),
           "planes to host");
      STEP(hipEventRecord(h->ev_sam, s), "event");
      STEP(hipEventSynchronize(h->ev_sam), "planes sync");
      const int cb = live->fn(live->user, (size_t)l, h->sam_planes_host, h->sam_idx_host);
      if (cb != 0)
        return c->fail(ULLIS_HIP_ERR_INVALID, "suffix automaton callback failed at layer " +
                                                  std::to_string(l) + " (" + std::to_string(cb) +
                                                  ")");
      STEP(hipMemcpyAsync(h->sam_idx_dev + l * nd, h->sam_idx_host, (size_t)nd,
                          hipMemcpyHostToDevice, s),
           "indices to device");
      STEP(rosa_expand_layers(s, h->sam_idx_dev + l * nd, h->e_host.data() + l, h->e_dev + l, 1, B,
                              T, D, h->y16 + l * nd, h->idx_rm + l * nd),
           "rosa y");
      const Block& bo = h->blocks[l];
      PackedFwdOut o;
      o.y32 = h->o_pre + l * nd;
      STEP(packed_forward(s, h->y16 + l * nd, kF16, R, D, D, bo.o.bits, bo.o.scale, bo.o.bias, o),
           "o");
    }
    float* ar = h->after_rosa + l * nd;
    // CMix (src/model.rs:1018-1078) on ar = x_l + o_l (add_inplace,
    // src/model.rs:2890), formed by the LN2 kernel
    uint16_t* ln2 = h->ln2_16 + l * nd;
    uint16_t* sh = h->shifted16 + l * nd;
    uint16_t* key = h->key16 + l * nf;
    uint16_t* r2 = h->relu2_16 + l * nf;
    if (!live) STEP(hipStreamWaitEvent(s, h->ev_o[l], 0), "event wait");
    PHASE_AT(s, kPhFwdLn);
    PROBED(ULLIS_HIP_PROBE_LN_FORWARD,
           layer_norm_mix_forward(s, h->o_pre + l * nd, R, T, D, b.ln2.w, b.ln2.b, ln2, true,
                                  b.cx_k, sh, nullptr, nullptr, nullptr, nullptr, x_l, ar),
           "ln2 + mix");
    PHASE_AT(s, kPhFwdCmix);
    {
      PackedFwdOut o;
      o.y16 = key;
      o.relu2_16 = r2;
      PROBED(ULLIS_HIP_PROBE_KEY_FORWARD,
             packed_forward(s, sh, kF16, R, D, F, b.key.bits, b.key.scale, nullptr, o), "key");
    }
    PROBED(ULLIS_HIP_PROBE_VALUE_FORWARD,
           fp16_forward(s, r2, kF16, R, F, D, b.value, h->resid + (l + 1) * nd, ar, nullptr),
           "value");
  }
  float* x_last = h->resid + L * nd;
  PHASE_AT(s, kPhFwdLn);
  STEP(layer_norm_forward(s, x_last, R, D, h->ln_out.w, h->ln_out.b, nullptr, h->ln16), "ln_out");
  PHASE_AT(s, kPhHead);

  // ------------------------------------------------------------ head + CE
  {
    // gradients only: the head's weight-gradient partials stay in gp_head
    // for the end-of-step update
    HeadCe hc{};
    hc.rows = R;
    hc.time = T;
    hc.d = D;
    hc.vocab = h->V;
    hc.hidden16 = h->ln16;
    hc.bits = h->head.bits;
    hc.bits_t = h->head.bits_t;
    hc.scale = h->head.scale;
    hc.bias = h->head.bias;
    hc.targets = labels;
    hc.ignore_id = ignore_id;
    hc.row_loss = rl;
    hc.stats = h->stats;  // the update jobs read gscale from here
    hc.stats2 = stats4;
    hc.g_hidden = h->g_a;
    hc.ste = ste;
    hc.gpart_all = h->gp_head;
    hc.invalid = h->invalid;  // labels >= vocab refuse the step's updates
    PROBED_SPAN(ULLIS_HIP_PROBE_HEAD_CE, head_ce(s, hc, h->head_ws), "head ce");
  }
  // LN_out backward (src/model.rs:2932-2937)
  PHASE_AT(s, kPhBwdLn);
  STEP(layer_norm_backward_rows(s, x_last, h->g_a, R, D, h->ln_out.w, h->g_x, 0, h->slots + L,
                                h->pt_lnout, &nb),
       "ln_out bwd");
  if (nb != h->nb_ln) return c->fail(ULLIS_HIP_ERR_RUNTIME, "ln_out backward partial count");
  // the head and LN_out gradients are complete: their updates run on the
  // second stream (nothing later in the step reads those parameters)
  STEP(hipEventRecord(h->ev_head, s), "event");
  STEP(hipStreamWaitEvent(h->side, h->ev_head, 0), "event wait");
  if (int rc = run_update_seg(h, h->side, (int)L, lr)) return rc;
  STEP(scale_to_f16(s, h->g_x, nd, h->slots + L, h->gx16_b + L * nd), "g_x fp16");

  // ------------------------------------------------------------ backward
  for (long l = L - 1; l >= 0; --l) {
    Block& b = h->blocks[l];
    const float* slot_in = h->slots + l + 1;
    float* slot_mid = h->slots + l;
    const uint16_t* ln2 = h->ln2_16 + l * nd;
    const uint16_t* sh = h->shifted16 + l * nd;
    const uint16_t* key = h->key16 + l * nf;
    const uint16_t* r2 = h->relu2_16 + l * nf;
    const float* ar = h->after_rosa + l * nd;
    const long pc = (long)h->nb_col * D;

    PHASE_AT(s, kPhBwdCmix);
    // CMix backward (src/model.rs:1145-1177): value input gradient (+ ReLU^2
    // backward into gk16) with the value weight gradient, then the key input
    // gradient with the key weight gradient
    {
      uint16_t* gx16_in = h->gx16_b + (l + 1) * nd;
      uint16_t* gk16 = h->gk16;
      const GradIn gx{h->g_x, slot_in, gx16_in};
      const GradIn g16_only{nullptr, slot_in};
      const WeightGradArgs vdw{g16_only, gx16_in, r2, R, F, D, h->splits_value,
                               h->gp_value + l * h->splits_value * D * F};
      const WeightGradArgs kdw{g16_only, gk16, sh, R, D, F, h->splits_key,
                               h->gp_key + l * h->splits_key * F * D};
      Fp16DxArgs vdx{gx, R, F, D, b.value, nullptr, key, gk16};
      vdx.w_t = b.value_t;
      PROBED(ULLIS_HIP_PROBE_VALUE_BACKWARD, fp16_backward_pair(s, vdx, vdw), "value backward");
      PROBED(ULLIS_HIP_PROBE_KEY_BACKWARD,
             packed_backward_pair(s,
                                  PackedDxArgs{g16_only, gk16, R, D, F, b.key.bits_t, b.key.scale,
                                               h->g_a, nullptr, 0},
                                  kdw),
             "key backward");
    }
    // CMix time-shift mix backward (x_k gradient) fused with the LN2
    // backward, += into g_x (src/model.rs:2958-2963)
    PHASE_AT(s, kPhBwdLn);
    {
      int nb_mix = 0;
      PROBED(ULLIS_HIP_PROBE_LN_BACKWARD,
             layer_norm_mix_backward_rows(s, ar, h->g_a, ln2, b.cx_k, R, T, D, b.ln2.w, h->g_x, 1,
                                          slot_mid, h->pt_ln2 + l * 2L * h->nb_ln * D,
                                          h->pt_mix + l * h->nb_mix * D, h->g_b, &nb, &nb_mix),
             "mix + ln2 bwd");
      if (nb != h->nb_ln || nb_mix != h->nb_mix)
        return c->fail(ULLIS_HIP_ERR_RUNTIME, "mix / ln2 backward partial count");
    }
    // O bias gradient (column sums of g_x) and the fp16 copy of g_x for the
    // O GEMMs here and the CMix GEMMs of the block below.
    uint16_t* gx16_l = h->gx16_b + l * nd;
    PHASE_AT(s, kPhBwdRosa);
    STEP(column_sum_partials(s, h->g_x, nullptr, R, D, h->pt_ob + l * pc, &nb, gx16_l, slot_mid),
         "o g_bias + g_x fp16");
    if (nb != h->nb_col) return c->fail(ULLIS_HIP_ERR_RUNTIME, "o bias partial count");

    // ROSA O stop-grad backward (src/model.rs:1491-1522) on the second
    // stream: the O weight gradient, and the O input gradient g_y reduced
    // straight to the e gradient partials (g_e = column sums of
    // g_y * (2 idx - 1); with stop_grad_bits nothing else reads g_y). It reads
    // only the fp16 gradient copy of this boundary and this layer's amax slot,
    // both final here.
    STEP(hipEventRecord(h->ev_bwd[l], s), "event");
    STEP(hipStreamWaitEvent(h->side, h->ev_bwd[l], 0), "event wait");
    {
      const GradIn g16_only{nullptr, slot_mid};
      PackedDxArgs dx{g16_only, gx16_l, R, D, D, b.o.bits_t, b.o.scale, h->g_side, nullptr, 0};
      dx.sign_idx = h->idx_rm + l * nd;
      dx.col_part = h->pt_e + l * pc;  // column_partial_blocks(R) groups of 16 rows
      PROBED(ULLIS_HIP_PROBE_O_BACKWARD,
             packed_backward_pair(h->side, dx,
                                  WeightGradArgs{g16_only, gx16_l, h->y16 + l * nd, R, D, D,
                                                 h->splits_o, h->gp_o + l * h->splits_o * D * D}),
             "o backward");
    }
    // every gradient of layer l is complete: its updates run on the second
    // stream too (nothing later in the step reads layer l's parameters)
    if (int rc = run_update_seg(h, h->side, (int)l, lr)) return rc;

    if (b.has_ln0) {  // (src/model.rs:2978-2982)
      PHASE_AT(s, kPhBwdLn);
      STEP(layer_norm_backward_rows(s, x_emb, h->g_x, R, D, b.ln0.w, g_emb, 0, nullptr, h->pt_ln0,
                                    &nb),
           "ln0 bwd");
      if (nb != h->nb_ln) {
        // another LN backward path (unaligned x_emb / g_emb): step LN0 here
        // and leave its batched job out
        ln0_now = true;
        STEP(layer_norm_param_finish(s, h->pt_ln0, nb, D, nullptr, nullptr, lr, b.ln0.w,
                                     b.ln0.w_res, b.ln0.b, b.ln0.b_res, h->invalid),
             "ln0 step");
      }
    } else if (l == 0) {
      STEP(copy_device(s, g_emb, h->g_x, (long)sizeof(float) * nd), "copy g_emb");
    }
  }

  if (emb) PHASE_AT(s, kPhEmbedSgd);
  if (emb)
    STEP(embedding_scatter_sgd(s, emb->table, emb->residual, emb->vocab, D, emb->tokens, R, g_emb,
                               lr, h->invalid),
         "embedding scatter sgd");
  // the second stream's work is done before the updates and the step's end
  // (its tail is the O backward and the updates: timed as bwd_rosa)
  PHASE_AT(s, kPhBwdRosa);
  STEP(hipEventRecord(h->ev_join, h->side), "event");
  STEP(hipStreamWaitEvent(s, h->ev_join, 0), "event wait");

  // ------------------------------------------------ end-of-step updates
  // LN0 (unless LN0 backward took the other path and stepped it already)
  if (!ln0_now)
    if (int rc = run_update_seg(h, s, (int)L + 1, lr)) return rc;
  for (const Packed* k : h->trans_generic)
    STEP(transpose_bits(s, k->bits, k->out, k->in, k->bits_t), "bits_t");
  if (invalid_out) STEP(copy_device(s, invalid_out, h->invalid, sizeof(uint32_t)), "invalid");
  PHASE_AT(s, kPhEnd);
  return 0;
}

// One step's arguments: a step from gathered rows (ullis_hip_heron_step) or
// from token ids (emb set: gather, step, scatter-SGD).
struct StepCall {
  const float* x_emb;
  const uint32_t* labels;
  uint32_t ignore_id;
  float lr;
  const uint8_t* rosa_idx;
  float* g_emb;
  float* row_loss;
  float* stats4;
  uint32_t* qkv_bits;
  uint32_t* invalid;
  bool from_tokens;
  EmbedArgs emb;
  const SamHandoff* live = nullptr;
  ullis_hip_heron::StepArgs key() const {
    ullis_hip_heron::StepArgs k{};
    const void* p[] = {x_emb,    labels,   rosa_idx,     g_emb,           row_loss,
                       stats4,   qkv_bits, invalid,      emb.table,       emb.residual,
                       emb.tokens};
    static_assert(sizeof(p) / sizeof(p[0]) == sizeof(k.p) / sizeof(k.p[0]), "step key");
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); ++i) k.p[i] = p[i];
    k.ignore_id = ignore_id;
    k.lr = lr;
    k.vocab = from_tokens ? emb.vocab : -1;
    return k;
  }
};

int step_call_launches(ullis_hip_heron* h, const StepCall& sc) {
  ullis_hip_ctx* c = h->ctx;
  if (!sc.from_tokens)
    return step_launches(h, sc.x_emb, sc.labels, sc.ignore_id, sc.lr, sc.rosa_idx, sc.g_emb,
                         sc.row_loss, sc.stats4, sc.qkv_bits, sc.invalid, nullptr, sc.live);
  // the refused-step counter starts the step here: the gather adds the token
  // ids >= vocab, the head the labels >= vocab
  PHASE_AT(c->stream, kPhEmbed);
  STEP(fill_f32(c->stream, reinterpret_cast<float*>(h->invalid), 1, 0.0f), "clear invalid");
  STEP(embedding_gather(c->stream, sc.emb.table, sc.emb.vocab, h->D, sc.emb.tokens, h->rows,
                        const_cast<float*>(sc.x_emb), h->invalid),
       "embedding gather");
  return step_launches(h, sc.x_emb, sc.labels, sc.ignore_id, sc.lr, sc.rosa_idx, sc.g_emb,
                       sc.row_loss, sc.stats4, sc.qkv_bits, sc.invalid, &sc.emb, sc.live);
}

// Eager launches, or (step graph on) the captured graph of them, captured
// again whenever the step's arguments change.
int run_step(ullis_hip_heron* h, const StepCall& sc) {
  ullis_hip_ctx* c = h->ctx;
  // probed steps run eagerly: the probe times individual launches; so do
  // steps with a live automaton, which synchronise with the host every layer
  if (!h->graph_on || h->probe != ULLIS_HIP_PROBE_NONE || t_launch_probe || sc.live ||
      h->phase_on)
    return step_call_launches(h, sc);
  const ullis_hip_heron::StepArgs args = sc.key();
  hipStream_t s = c->stream;
  if (!h->graph_exec || !(args == h->graph_args)) {
    if (h->graph_exec) {
      // the previous graph may still be running
      STEP(hipStreamSynchronize(s), "graph sync");
      STEP(hipGraphExecDestroy(h->graph_exec), "graph destroy");
      h->graph_exec = nullptr;
    }
    STEP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "graph capture");
    const int rc = step_call_launches(h, sc);
    hipGraph_t g = nullptr;
    const hipError_t end = hipStreamEndCapture(s, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (int rc2 = c->hip(end, "graph capture end")) return rc2;
    const hipError_t inst = hipGraphInstantiate(&h->graph_exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (int rc2 = c->hip(inst, "graph instantiate")) {
      h->graph_exec = nullptr;
      return rc2;
    }
    h->graph_args = args;
  }
  STEP(hipGraphLaunch(h->graph_exec, s), "graph launch");
  return 0;
}

}  // namespace

extern "C" {

int ullis_hip_heron_step_tokens(ullis_hip_heron* h, uint16_t* table, float* table_residual,
                                size_t vocab, const uint32_t* tokens, const uint32_t* labels,
                                uint32_t ignore_id, float lr, const uint8_t* rosa_idx,
                                float* x_emb, float* g_emb, float* row_loss, float* stats4,
                                uint32_t* qkv_bits, uint32_t* invalid) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  if (!table || !table_residual || !tokens || !labels || !rosa_idx || !x_emb || !g_emb)
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "heron step from tokens needs the table, its carry, tokens, labels, rosa_idx, "
                   "x_emb and g_emb");
  if (vocab == 0 || vocab > (size_t)UINT32_MAX)
    return c->fail(ULLIS_HIP_ERR_INVALID, "embedding vocab must be non-zero and fit u32");
  if (!(lr > 0.0f) || !__builtin_isfinite(lr))
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "train step requires a positive learning rate and time >= 2");
  const StepCall sc{x_emb,    labels, ignore_id, lr,   rosa_idx,
                    g_emb,    row_loss, stats4, qkv_bits, invalid,
                    true,     EmbedArgs{table, table_residual, (long)vocab, tokens}};
  return run_step(h, sc);
}

int ullis_hip_heron_set_graph(ullis_hip_heron* h, int enable) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  h->graph_on = enable != 0;
  if (h->graph_exec) {
    STEP(hipStreamSynchronize(c->stream), "graph sync");
    STEP(hipGraphExecDestroy(h->graph_exec), "graph destroy");
    h->graph_exec = nullptr;
  }
  return 0;
}

int ullis_hip_heron_step(ullis_hip_heron* h, const float* x_emb, const uint32_t* labels,
                         uint32_t ignore_id, float lr, const uint8_t* rosa_idx, float* g_emb,
                         float* row_loss, float* stats4, uint32_t* qkv_bits, uint32_t* invalid) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  if (!x_emb || !labels || !rosa_idx || !g_emb)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron step needs x_emb, labels, rosa_idx and g_emb");
  if (!(lr > 0.0f) || !__builtin_isfinite(lr))
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "train step requires a positive learning rate and time >= 2");
  const StepCall sc{x_emb,  labels,   ignore_id, lr,    rosa_idx, g_emb,
                    row_loss, stats4, qkv_bits,  invalid, false,  EmbedArgs{}};
  return run_step(h, sc);
}

int ullis_hip_heron_step_sam(ullis_hip_heron* h, uint16_t* table, float* table_residual,
                             size_t vocab, const uint32_t* tokens, float* x_emb,
                             const uint32_t* labels, uint32_t ignore_id, float lr,
                             ullis_hip_sam_fn sam, void* sam_user, float* g_emb, float* row_loss,
                             float* stats4, uint32_t* qkv_bits, uint32_t* invalid) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  if (!x_emb || !labels || !g_emb || !sam)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron step with an automaton needs x_emb, labels, "
                                          "g_emb and the automaton callback");
  if (table && (!table_residual || !tokens || vocab == 0 || vocab > (size_t)UINT32_MAX))
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "heron step from tokens needs the table carry, tokens and a u32 vocab");
  if (!(lr > 0.0f) || !__builtin_isfinite(lr))
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "train step requires a positive learning rate and time >= 2");
  const long nd = h->rows * h->D;
  if (!h->sam_idx_dev) {
    // first live step: pinned staging of one layer's planes and indices, and
    // device indices of every layer
    const size_t words = (size_t)cdiv(nd, 32);
    if (hipHostMalloc(reinterpret_cast<void**>(&h->sam_planes_host), 4 * 3 * words,
                      hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&h->sam_idx_host), (size_t)nd,
                      hipHostMallocDefault) != hipSuccess ||
        hipMalloc(&h->sam_idx_dev, (size_t)nd * h->L) != hipSuccess ||
        hipEventCreateWithFlags(&h->ev_sam, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      return c->fail(ULLIS_HIP_ERR_NOMEM, "suffix automaton staging allocation failed");
    }
  }
  const SamHandoff live{sam, sam_user};
  StepCall sc{x_emb, labels, ignore_id, lr, h->sam_idx_dev, g_emb, row_loss, stats4, qkv_bits,
              invalid, table != nullptr,
              table ? EmbedArgs{table, table_residual, (long)vocab, tokens} : EmbedArgs{}};
  sc.live = &live;
  return run_step(h, sc);
}

int ullis_hip_heron_decode_init(ullis_hip_heron* h, size_t batch, int flags) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  if ((flags & ~ULLIS_HIP_DECODE_EAGER) != 0)
    return c->fail(ULLIS_HIP_ERR_INVALID, "unknown decode flags");
  if (batch == 0 || batch > (size_t)kGemvMaxRows)
    return c->fail(ULLIS_HIP_ERR_INVALID, "decode batch must be in [1, 8]");
  auto& d = h->dec;
  const long B = (long)batch, D = h->D, F = h->F, L = h->L;
  const long words = cdiv(B * D, 32);
  if (d.batch != B) {
    STEP(hipStreamSynchronize(c->stream), "decode sync");
    for (auto& g : d.graph)
      if (g) (void)hipGraphExecDestroy(g);
    if (d.mem) (void)hipFree(d.mem);
    if (d.planes_host) (void)hipHostFree(d.planes_host);
    if (d.idx_host) (void)hipHostFree(d.idx_host);
    d = ullis_hip_heron::Decode{};
    // one carving sequence, run once to size the allocation and once to place the buffers
    auto carve = [&](auto& cv) {
      d.rosa_prev = cv.template take<float>(2 * L * B * D);
      d.cmix_prev = cv.template take<float>(2 * L * B * D);
      d.x = cv.template take<float>(B * D);
      d.x2 = cv.template take<float>(B * D);
      d.ln = cv.template take<float>(B * D);
      d.q = cv.template take<float>(B * D);
      d.k = cv.template take<float>(B * D);
      d.v = cv.template take<float>(B * D);
      d.q16 = cv.template take<uint16_t>(B * D);
      d.k16 = cv.template take<uint16_t>(B * D);
      d.v16 = cv.template take<uint16_t>(B * D);
      d.y16 = cv.template take<uint16_t>(B * D);
      d.sh16 = cv.template take<uint16_t>(B * D);
      d.hid16 = cv.template take<uint16_t>(B * D);
      d.key16 = cv.template take<uint16_t>(B * F);
      d.r2_16 = cv.template take<uint16_t>(B * F);
      d.idx = cv.template take<uint8_t>(B * D);
      d.idx_rm = cv.template take<uint8_t>(B * D);
      d.planes = cv.template take<uint32_t>(3 * words);
    };
    CarveSizer sizer;
    carve(sizer);
    if (hipMalloc(&d.mem, sizer.used) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&d.planes_host), 4ul * 3 * words,
                      hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&d.idx_host), (size_t)(B * D),
                      hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      return c->fail(ULLIS_HIP_ERR_NOMEM, "decode state allocation failed");
    }
    Carver cv(d.mem);
    carve(cv);
    d.batch = B;
  }
  // new sequences: no previous token, i.e. previous LayerNorm outputs of 0
  // (time_shift_one then gives -x)
  STEP(fill_f32(c->stream, d.rosa_prev, L * B * D, 0.0f), "decode state clear");
  STEP(fill_f32(c->stream, d.cmix_prev, L * B * D, 0.0f), "decode state clear");
  d.parity = 0;
  d.eager = (flags & ULLIS_HIP_DECODE_EAGER) != 0;
  return 0;
}

}  // extern "C"

namespace {

struct DecodeCall {
  const uint16_t* table;
  long vocab;
  const uint32_t* tokens;
  const uint8_t* rosa_idx;
  ullis_hip_sam_fn sam;
  void* sam_user;
  float* logits;
  uint32_t* next;
  uint32_t* invalid;
  ullis_hip_heron::Decode::Key key() const {
    return {{table, tokens, rosa_idx, logits, next, invalid}, vocab};
  }
};

// The launches of one decode token, reading the previous-token buffers of
// `parity`: generate_step (src/model.rs:2717-2753), every block's
// forward_one (src/model.rs:2243-2262), the head and the argmax.
int decode_launches(ullis_hip_heron* h, const DecodeCall& a, int parity) {
  ullis_hip_ctx* c = h->ctx;
  auto& d = h->dec;
  hipStream_t s = c->stream;
  const long B = d.batch, D = h->D, F = h->F, V = h->V, L = h->L;
  const long nd = B * D, words = cdiv(nd, 32);
  const bool fused = decode_fused_ok(B, D, F);
  float* rp_in = d.rosa_prev + parity * L * nd;
  float* rp_out = d.rosa_prev + (1 - parity) * L * nd;
  float* cp_in = d.cmix_prev + parity * L * nd;
  float* cp_out = d.cmix_prev + (1 - parity) * L * nd;
  const Block& b0 = h->blocks[0];
  // x = emb(token); h = ln0(x) at the first block
  const bool ln0_fused = fused;  // the embedding kernel applies LN0 where the fused kernels apply
  STEP(decode_embed(s, a.table, a.vocab, D, a.tokens, B, d.x, a.invalid,
                    b0.has_ln0 && ln0_fused ? b0.ln0.w : nullptr,
                    b0.has_ln0 && ln0_fused ? b0.ln0.b : nullptr),
       "decode embed");
  if (b0.has_ln0 && !ln0_fused) {
    STEP(layer_norm_forward(s, d.x, B, D, b0.ln0.w, b0.ln0.b, d.ln, nullptr), "ln0");
    STEP(copy_device(s, d.x, d.ln, 4l * nd), "ln0 copy");
  }
  for (long l = 0; l < L; ++l) {
    const Block& b = h->blocks[l];
    // ROSA forward_one (src/model.rs:1320-1353): the Q/K/V sign planes of
    // mix(LN3(h)) (bit_from_activation, src/rosa.rs:372)
    DecodeQkv p;
    DecodeO po;
    if (fused) {
      const Packed* lin[3] = {&b.q, &b.k, &b.v};
      const uint16_t* mix[3] = {b.x_q, b.x_k, b.x_v};
      for (int j = 0; j < 3; ++j) {
        p.mix[j] = mix[j];
        p.bits[j] = lin[j]->bits;
        p.scale[j] = lin[j]->scale;
        p.bias[j] = lin[j]->bias;
        p.planes[j] = d.planes + j * words;
      }
      po.idx = a.rosa_idx ? a.rosa_idx + l * nd : d.idx;
      po.e = b.e;
      po.bits = b.o.bits;
      po.scale = b.o.scale;
      po.bias = b.o.bias;
      // with the indices given, Q/K/V and O in one launch; a live automaton
      // needs this token's Q/K/V planes first
      STEP(decode_qkvo(s, d.x, d.x2, B, D, a.sam ? 0 : 2, b.ln3.w, b.ln3.b, rp_in + l * nd,
                       rp_out + l * nd, p, po),
           "decode qkv");
    } else {
      STEP(layer_norm_forward(s, d.x, B, D, b.ln3.w, b.ln3.b, d.ln, nullptr), "ln3");
      STEP(decode_mix(s, d.ln, rp_in + l * nd, rp_out + l * nd, B, D, b.x_q, d.q16, b.x_k,
                      d.k16, b.x_v, d.v16),
           "rosa mixes");
      PackedFwdOut oq, ok, ov;
      oq.y32 = d.q;
      ok.y32 = d.k;
      ov.y32 = d.v;
      STEP(packed_forward(s, d.q16, kF16, B, D, D, b.q.bits, b.q.scale, b.q.bias, oq), "q");
      STEP(packed_forward(s, d.k16, kF16, B, D, D, b.k.bits, b.k.scale, b.k.bias, ok), "k");
      STEP(packed_forward(s, d.v16, kF16, B, D, D, b.v.bits, b.v.scale, b.v.bias, ov), "v");
      STEP(sign_pack_bits(s, d.q, nd, d.planes), "q bits");
      STEP(sign_pack_bits(s, d.k, nd, d.planes + words), "k bits");
      STEP(sign_pack_bits(s, d.v, nd, d.planes + 2 * words), "v bits");
    }
    const uint8_t* idx = a.rosa_idx ? a.rosa_idx + l * nd : d.idx;
    if (a.sam) {
      STEP(hipMemcpyAsync(d.planes_host, d.planes, 4ul * 3 * words, hipMemcpyDeviceToHost, s),
           "planes to host");
      STEP(hipStreamSynchronize(s), "planes sync");
      const int cb = a.sam(a.sam_user, (size_t)l, d.planes_host, d.idx_host);
      if (cb != 0)
        return c->fail(ULLIS_HIP_ERR_INVALID, "suffix automaton callback failed at layer " +
                                                  std::to_string(l) + " (" + std::to_string(cb) +
                                                  ")");
      STEP(hipMemcpyAsync(d.idx, d.idx_host, (size_t)nd, hipMemcpyHostToDevice, s),
           "indices to device");
    }
    // h += O((2 idx - 1) e); the fused path leaves it in x2
    if (fused) {
      if (a.sam)
        STEP(decode_qkvo(s, d.x, d.x2, B, D, 1, b.ln3.w, b.ln3.b, rp_in + l * nd,
                         rp_out + l * nd, p, po),
             "decode o");
    } else {
      STEP(rosa_expand(s, idx, b.e, B, 1, D, d.y16, d.idx_rm), "rosa y");
      PackedFwdOut o;
      o.y32 = d.x;
      o.resid = d.x;
      STEP(packed_forward(s, d.y16, kF16, B, D, D, b.o.bits, b.o.scale, b.o.bias, o), "o");
    }
    // CMix forward_one (src/model.rs:1003-1016): h += value(relu2(key(mix(ln2(h)))))
    if (fused) {
      STEP(decode_key(s, d.x2, B, D, F, b.ln2.w, b.ln2.b, cp_in + l * nd, cp_out + l * nd,
                      b.cx_k, b.key.bits, b.key.scale, d.r2_16),
           "decode key");
    } else {
      STEP(layer_norm_forward(s, d.x, B, D, b.ln2.w, b.ln2.b, d.ln, nullptr), "ln2");
      STEP(decode_mix(s, d.ln, cp_in + l * nd, cp_out + l * nd, B, D, b.cx_k, d.sh16, nullptr,
                      nullptr, nullptr, nullptr),
           "cmix mix");
      PackedFwdOut o;
      o.y16 = d.key16;  // the products write relu2 beside the key itself
      o.relu2_16 = d.r2_16;
      STEP(packed_forward(s, d.sh16, kF16, B, D, F, b.key.bits, b.key.scale, nullptr, o), "key");
    }
    STEP(fp16_forward(s, d.r2_16, kF16, B, F, D, b.value, d.x, fused ? d.x2 : d.x, nullptr),
         "value");
  }
  if (fused) {
    STEP(decode_head(s, d.x, B, D, V, h->ln_out.w, h->ln_out.b, h->head.bits, h->head.scale,
                     h->head.bias, a.logits),
         "decode head");
  } else {
    STEP(layer_norm_forward(s, d.x, B, D, h->ln_out.w, h->ln_out.b, nullptr, d.hid16), "ln_out");
    PackedFwdOut o;
    o.y32 = a.logits;
    STEP(packed_forward(s, d.hid16, kF16, B, D, V, h->head.bits, h->head.scale, h->head.bias, o),
         "head");
  }
  if (a.next) STEP(argmax_rows(s, a.logits, B, V, a.next), "argmax");
  return 0;
}

}  // namespace

extern "C" {

int ullis_hip_heron_decode_step(ullis_hip_heron* h, const uint16_t* table, size_t vocab,
                                const uint32_t* tokens, const uint8_t* rosa_idx,
                                ullis_hip_sam_fn sam, void* sam_user, float* logits,
                                uint32_t* next_tokens, uint32_t* invalid) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  auto& d = h->dec;
  if (!d.mem) return c->fail(ULLIS_HIP_ERR_INVALID, "decode step before ullis_hip_heron_decode_init");
  if (!table || !tokens || !logits || vocab == 0 || vocab > (size_t)UINT32_MAX)
    return c->fail(ULLIS_HIP_ERR_INVALID, "decode step needs the table, tokens and logits");
  if ((rosa_idx == nullptr) == (sam == nullptr))
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "decode step takes either the automaton's indices or its callback");
  const DecodeCall a{table, (long)vocab, tokens, rosa_idx, sam, sam_user, logits, next_tokens,
                     invalid};
  const int par = d.parity;
  if (sam || t_launch_probe || d.eager) {
    // a live automaton synchronises with the host every layer: eager launches
    if (int rc = decode_launches(h, a, par)) return rc;
  } else {
    hipStream_t s = c->stream;
    const auto key = a.key();
    if (!d.graph[par] || !(d.graph_key[par] == key)) {
      if (d.graph[par]) {
        STEP(hipStreamSynchronize(s), "decode graph sync");
        STEP(hipGraphExecDestroy(d.graph[par]), "decode graph destroy");
        d.graph[par] = nullptr;
      }
      STEP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "decode graph capture");
      const int rc = decode_launches(h, a, par);
      hipGraph_t g = nullptr;
      const hipError_t end = hipStreamEndCapture(s, &g);
      if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
      }
      if (int rc2 = c->hip(end, "decode graph capture end")) return rc2;
      const hipError_t inst = hipGraphInstantiate(&d.graph[par], g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (int rc2 = c->hip(inst, "decode graph instantiate")) {
        d.graph[par] = nullptr;
        return rc2;
      }
      d.graph_key[par] = key;
    }
    STEP(hipGraphLaunch(d.graph[par], s), "decode graph launch");
  }
  d.parity = 1 - par;
  return 0;
}

int ullis_hip_heron_causal_loss(ullis_hip_heron* h, const float* g_emb, const uint32_t* labels,
                                uint32_t ignore_id, const float* row_loss,
                                const float* table_residual, size_t table_elems,
                                ullis_hip_causal_loss* out) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  if (!g_emb || !labels || !out)
    return c->fail(ULLIS_HIP_ERR_INVALID, "causal_loss needs g_emb, labels and out");
  if (table_elems > 0 && !table_residual)
    return c->fail(ULLIS_HIP_ERR_INVALID, "causal_loss: table_elems without table_residual");
  const long R = h->rows, D = h->D, F = h->F, V = h->V, L = h->L;
  auto task = [](int kind, int field, int rms, const void* p, long n, long denom) {
    return DiagTask{kind, field, rms, p, n, denom};
  };
  const DiagTask tasks[] = {
      task(DiagTask::kSqF32, kDiagEmbedGradRms, 1, g_emb, R * D, R * D),
      task(DiagTask::kSqF32, kDiagHeadScaleGradRms, 1, h->gscale_head, V, V),
      task(DiagTask::kSqF16, kDiagHeadScaleRms, 1, h->head.scale, V, V),
      task(DiagTask::kAbsF32, kDiagResidualAbsMean, 0, table_residual, (long)table_elems,
           (long)table_elems),
      task(DiagTask::kSqF16, kDiagCmixValueRms, 1, h->blocks[0].value, D * F, D * F),
      task(DiagTask::kAbsF16, kDiagHeadLatentAbsMean, 0, h->head.latent, V * D, V * D),
      task(DiagTask::kSumF32, kDiagHeadLatentStepAbs, 0, h->step_head, V, V * D),
      task(DiagTask::kSqF16, kDiagHeadBiasRms, 1, h->head.bias, V, V),
      task(DiagTask::kSumU32, kDiagFlipsHead, 0, h->flips_head, V, V),
      task(DiagTask::kSumU32, kDiagFlipsCmix, 0, h->flips_key, L * F, L * F),
      task(DiagTask::kSumU32, kDiagFlipsRosaO, 0, h->flips_o, L * D, L * D),
  };
  DiagArgs a{row_loss ? row_loss : h->row_loss, labels, R, h->time, V, ignore_id, h->stats, out};
  STEP(causal_loss_diag(c->stream, a, tasks, (int)(sizeof(tasks) / sizeof(tasks[0])), h->diag_ws),
       "causal loss");
  return 0;
}

}  // extern "C"
