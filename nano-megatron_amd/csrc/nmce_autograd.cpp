// The drop-in loss's one-pass path at TP = 1 as a C++ autograd node.
//
// Forward and backward of cross_entropy.py:16-65 followed by the wrapper's
// .mean() (:85), for the rows the one-pass kernel takes: one launch of
// nmce_ce_fwd_bwd writes the per-token loss, the row statistics and the
// gradient of the mean for the assumed upstream value; the backward launches
// nmce_ce_grad_rescale_unless (gradient in the logits' storage) or
// nmce_ce_bwd_scaled_unless (a separate buffer), which leave it as it is when
// the upstream value is the assumed one. Host code only: the kernels are
// libnmce.so's, reached through its C ABI (include/nmce.h).
//
// A node written in Python costs the autograd engine a hand-over to the
// interpreter on its device thread for every backward, and the forward's
// Python bookkeeping besides: tens of microseconds per call, which a small
// batch (a step of a few tens of microseconds of kernels) pays in full. The
// Python wrapper still validates the arguments and resolves the upstream
// hint; the target check of cross_entropy.py:79-81 runs here too
// (one_pass_mean_checked).
#include <torch/extension.h>
#include <torch/csrc/autograd/variable.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <chrono>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "nmce.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

void check(int status, const char* what) {
  TORCH_CHECK(status == 0, "nmce: ", what, " failed with status ", status, ": ",
              nmce_status_string(status));
}

int dtype_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kFloat) return NMCE_F32;
  if (t.scalar_type() == at::kBFloat16) return NMCE_BF16;
  TORCH_CHECK(false, "nmce: unsupported logits dtype ", t.scalar_type());
  return -1;
}

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Optional per-launch timing: HIP event pairs recorded on the launch stream
// around every launch of this file while enabled, read back by
// take_timeline() (the benchmark's per-call times).
std::mutex g_timeline_lock;
std::atomic<bool> g_timing{false};
std::vector<std::tuple<std::string, hipEvent_t, hipEvent_t>> g_timeline;

template <typename Launch>
void timed(const char* name, hipStream_t st, Launch&& launch) {
  if (!g_timing) {
    check(launch(), name);
    return;
  }
  hipEvent_t a = nullptr, b = nullptr;
  const bool made = hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess;
  if (!made || hipEventRecord(a, st) != hipSuccess) {
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    TORCH_CHECK(false, "nmce: creating or recording a timing event failed");
  }
  const int status = launch();
  if (hipEventRecord(b, st) != hipSuccess) {
    (void)hipEventSynchronize(a);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    check(status, name);
    TORCH_CHECK(false, "nmce: recording a timing event failed");
  }
  {
    std::lock_guard<std::mutex> g(g_timeline_lock);
    g_timeline.emplace_back(name, a, b);
  }
  check(status, name);
}

struct OnePassMean : public torch::autograd::Function<OnePassMean> {
  // logits [..., V] viewable as [rows, V] (16-byte aligned rows, V a whole
  // number of 16-byte vectors within the kernel's width; the wrapper checked),
  // target the flat contiguous int64 targets, hint the one-element fp32
  // upstream value to assume, bad_flag the address of the target check's
  // device word (0 without a check; not an autograd input), inplace whether
  // the gradient goes into the logits' storage.
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& logits,
                            const at::Tensor& target, const at::Tensor& hint, int64_t bad_flag,
                            bool inplace, int64_t vocab_start) {
    const c10::DeviceGuard device_guard(logits.device());
    const int64_t V = logits.size(-1);
    const at::Tensor rows = logits.view({-1, V});
    const int64_t n = rows.size(0);
    const int64_t ld = n > 1 ? rows.stride(0) : V;
    const int code = dtype_code(rows);
    at::Tensor out = at::empty({3, n}, rows.options().dtype(at::kFloat));  // loss, max, sum - 1
    at::Tensor loss = out.select(0, 0);
    at::Tensor row_stat = out.slice(0, 1, 3);
    at::Tensor grad = inplace ? rows : at::empty({n, V}, rows.options());
    const int64_t ldg = inplace ? ld : V;
    at::Tensor assumed = at::empty({1}, out.options());
    hipStream_t st = stream_of(rows);
    float* stats = out.data_ptr<float>();
    timed("nmce_ce_fwd_bwd", st, [&] {
      return nmce_ce_fwd_bwd(rows.data_ptr(), grad.data_ptr(), code, n, V, ld, ldg,
                             target.data_ptr<int64_t>(), stats, stats + n, stats + 2 * n,
                             hint.data_ptr<float>(), assumed.data_ptr<float>(),
                             reinterpret_cast<const int32_t*>(bad_flag),
                             static_cast<float>(n), st);
    });
    ctx->saved_data["inplace"] = inplace;
    ctx->saved_data["ld"] = ld;
    ctx->saved_data["vocab_start"] = vocab_start;
    ctx->saved_data["handed_out"] = false;
    ctx->saved_data["shape"] = logits.sizes().vec();
    if (inplace) {
      // The logits now hold the gradient: autograd nodes that saved them fail
      // their version check rather than read it.
      torch::autograd::impl::bump_version(logits);
      ctx->saved_data["grad_buf"] = logits.detach();
      ctx->save_for_backward({target, row_stat, assumed, hint});
    } else {
      ctx->save_for_backward({rows, target, row_stat, grad, assumed, hint});
    }
    return loss.mean();
  }

  static variable_list backward(AutogradContext* ctx, variable_list grad_outputs) {
    const c10::DeviceGuard device_guard(grad_outputs[0].device());
    at::Tensor go = grad_outputs[0].reshape({1});
    if (go.scalar_type() != at::kFloat) go = go.to(at::kFloat);
    go = go.contiguous();
    const bool inplace = ctx->saved_data["inplace"].toBool();
    const int64_t ld = ctx->saved_data["ld"].toInt();
    const std::vector<int64_t> shape = ctx->saved_data["shape"].toIntVector();
    const int64_t V = shape.back();
    const variable_list saved = ctx->get_saved_variables();
    variable_list grads(6);
    if (inplace) {
      TORCH_CHECK(!ctx->saved_data["handed_out"].toBool(),
                  "nmce: a second backward through an in-place one-pass loss needs the logits, "
                  "which now hold the gradient; pass inplace=False to differentiate it twice");
      const at::Tensor& target = saved[0];
      const at::Tensor& assumed = saved[2];
      const at::Tensor& hint = saved[3];
      at::Tensor grad = ctx->saved_data["grad_buf"].toTensor();
      const int64_t n = target.numel();
      hipStream_t st = stream_of(grad);
      timed("nmce_ce_grad_rescale_unless", st, [&] {
        return nmce_ce_grad_rescale_unless(grad.data_ptr(), dtype_code(grad), n, V, ld,
                                           go.data_ptr<float>(), assumed.data_ptr<float>(),
                                           hint.data_ptr<float>(), st);
      });
      ctx->saved_data["handed_out"] = true;
      ctx->saved_data["grad_buf"] = at::Tensor();
      grads[0] = grad;
      return grads;
    }
    const at::Tensor& rows = saved[0];
    const at::Tensor& target = saved[1];
    const at::Tensor& row_stat = saved[2];
    const at::Tensor& grad = saved[3];
    const at::Tensor& assumed = saved[4];
    const at::Tensor& hint = saved[5];
    const int64_t n = rows.size(0);
    const int64_t vocab_start = ctx->saved_data["vocab_start"].toInt();
    const float gdiv = static_cast<float>(n > 1 ? n : 1);
    hipStream_t st = stream_of(rows);
    const float* stats = row_stat.data_ptr<float>();
    if (ctx->saved_data["handed_out"].toBool()) {
      // A second backward through the same graph: the first one's buffer
      // belongs to its consumers; a new one from the logits.
      at::Tensor fresh = at::empty({n, V}, rows.options());
      timed("nmce_ce_bwd_scaled", st, [&] {
        return nmce_ce_bwd_scaled(rows.data_ptr(), fresh.data_ptr(), dtype_code(rows), n, V, ld,
                                  V, target.data_ptr<int64_t>(), vocab_start, stats, stats + n,
                                  go.data_ptr<float>(), 0, gdiv, st);
      });
      grads[0] = fresh.view(shape);
      return grads;
    }
    timed("nmce_ce_bwd_scaled_unless", st, [&] {
      return nmce_ce_bwd_scaled_unless(rows.data_ptr(), grad.data_ptr(), dtype_code(rows), n, V,
                                       ld, V, target.data_ptr<int64_t>(), vocab_start, stats,
                                       stats + n, go.data_ptr<float>(), gdiv,
                                       assumed.data_ptr<float>(), hint.data_ptr<float>(), st);
    });
    ctx->saved_data["handed_out"] = true;
    grads[0] = grad.view(shape);
    return grads;
  }
};

// ---- the target check ------------------------------------------------------
// nmce_validate_targets_once counts the targets outside [0, vocab) into a
// pinned host word (for the ValueError) and a device word that the one-pass
// kernel reads before its first store (it writes nothing when it is nonzero),
// on the loss stream just before the kernel. The host waits for the check's
// event after enqueueing the kernel, so the GPU starts on the loss meanwhile.

// The device word per (device, stream): the check and the kernel run on that
// stream one after the other, so calls on one stream can share it.
std::mutex g_flag_lock;
std::map<std::pair<int, hipStream_t>, at::Tensor> g_flags;

at::Tensor flag_word(const at::Tensor& like, hipStream_t st) {
  std::lock_guard<std::mutex> g(g_flag_lock);
  auto key = std::make_pair(static_cast<int>(like.device().index()), st);
  auto it = g_flags.find(key);
  if (it == g_flags.end())
    it = g_flags.emplace(key, at::empty({1}, like.options().dtype(at::kInt))).first;
  return it->second;
}

// Pinned count words with their events, pooled and reused once a check has
// been waited for (the kernel writes the word through its host mapping).
struct CheckSlot {
  at::Tensor host;
  hipEvent_t event = nullptr;
};
std::mutex g_slot_lock;
std::vector<CheckSlot> g_slots;

CheckSlot take_slot() {
  {
    std::lock_guard<std::mutex> g(g_slot_lock);
    if (!g_slots.empty()) {
      CheckSlot s = g_slots.back();
      g_slots.pop_back();
      return s;
    }
  }
  CheckSlot s;
  s.host = at::empty({1}, at::TensorOptions().dtype(at::kInt).pinned_memory(true));
  TORCH_CHECK(hipEventCreateWithFlags(&s.event, hipEventDisableTiming) == hipSuccess,
              "nmce: hipEventCreateWithFlags failed");
  return s;
}

// Waits for a recorded check on every way out of the call (the kernel writes
// the pinned word until then), and gives the slot back.
class CheckGuard {
 public:
  explicit CheckGuard(CheckSlot s) : slot_(std::move(s)) {}
  int32_t* host() { return slot_.host.data_ptr<int32_t>(); }
  hipEvent_t event() const { return slot_.event; }
  void recorded() { recorded_ = true; }
  // The count, once the check has finished. Polls first (the count is
  // usually there within microseconds of the launch), then blocks.
  int32_t wait() {
    if (recorded_) {
      pybind11::gil_scoped_release nogil;
      const auto until = std::chrono::steady_clock::now() + std::chrono::microseconds(200);
      hipError_t q = hipEventQuery(slot_.event);
      while (q == hipErrorNotReady && std::chrono::steady_clock::now() < until)
        q = hipEventQuery(slot_.event);
      if (q == hipErrorNotReady) q = hipEventSynchronize(slot_.event);
      recorded_ = false;
      TORCH_CHECK(q == hipSuccess, "nmce: waiting for the target check failed: ",
                  hipGetErrorString(q));
    }
    return *static_cast<volatile int32_t*>(slot_.host.data_ptr<int32_t>());
  }
  ~CheckGuard() {
    if (recorded_) (void)hipEventSynchronize(slot_.event);
    std::lock_guard<std::mutex> g(g_slot_lock);
    g_slots.push_back(std::move(slot_));
  }

 private:
  CheckSlot slot_;
  bool recorded_ = false;
};

at::Tensor one_pass_mean(const at::Tensor& logits, const at::Tensor& target,
                         const at::Tensor& hint, const c10::optional<at::Tensor>& bad_flag,
                         bool inplace, int64_t vocab_start) {
  const int64_t flag = bad_flag.has_value() && bad_flag->defined()
                           ? reinterpret_cast<int64_t>(bad_flag->data_ptr<int32_t>())
                           : 0;
  return OnePassMean::apply(logits, target, hint, flag, inplace, vocab_start);
}

// one_pass_mean with the target check of cross_entropy.py:79-81 in front:
// raises the reference's ValueError, after the kernel has left everything as
// it was, when a target lies outside [0, vocab_total).
at::Tensor one_pass_mean_checked(const at::Tensor& logits, const at::Tensor& target,
                                 const at::Tensor& hint, int64_t vocab_total, bool inplace,
                                 int64_t vocab_start) {
  const c10::DeviceGuard device_guard(logits.device());
  hipStream_t st = stream_of(logits);
  const at::Tensor flag = flag_word(logits, st);
  CheckGuard guard(take_slot());
  check(nmce_validate_targets_once(target.data_ptr<int64_t>(), target.numel(), vocab_total,
                                   guard.host(), flag.data_ptr<int32_t>(), st),
        "nmce_validate_targets_once");
  if (hipEventRecord(guard.event(), st) != hipSuccess) {
    // The check may still write the slot's word: let it finish first.
    (void)hipStreamSynchronize(st);
    TORCH_CHECK(false, "nmce: hipEventRecord failed");
  }
  guard.recorded();
  at::Tensor loss = OnePassMean::apply(logits, target, hint,
                                       reinterpret_cast<int64_t>(flag.data_ptr<int32_t>()),
                                       inplace, vocab_start);
  if (guard.wait() != 0)
    throw pybind11::value_error("target token id is outside the model vocabulary");
  return loss;
}

// The assumed upstream value a one-pass loss's forward used, for tests that
// follow which backward kept the forward's gradient: the saved fp32 word.
at::Tensor assumed_of(const at::Tensor& loss) {
  auto fn = loss.grad_fn();
  TORCH_CHECK(fn, "nmce: not a one-pass loss");
  auto* node = dynamic_cast<torch::autograd::CppNode<OnePassMean>*>(fn.get());
  TORCH_CHECK(node, "nmce: not a one-pass loss");
  const variable_list saved = node->ctx_.get_saved_variables();
  return saved[node->ctx_.saved_data.at("inplace").toBool() ? 2 : 4];
}

void set_timing(bool on) { g_timing = on; }

// (name, milliseconds) of every launch timed since the last call, in launch
// order; waits for the last of them.
std::vector<std::tuple<std::string, double>> take_timeline() {
  std::vector<std::tuple<std::string, hipEvent_t, hipEvent_t>> events;
  {
    std::lock_guard<std::mutex> g(g_timeline_lock);
    events.swap(g_timeline);
  }
  std::vector<std::tuple<std::string, double>> out;
  bool ok = true;
  for (auto& [name, a, b] : events) {
    float ms = 0.0f;
    ok = ok && hipEventSynchronize(b) == hipSuccess &&
         hipEventElapsedTime(&ms, a, b) == hipSuccess;
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    out.emplace_back(name, ms);
  }
  TORCH_CHECK(ok, "nmce: reading a launch's HIP events failed");
  return out;
}

// For measurements (no counterpart in the reference): an autograd node that
// stands where the LM-head matmul is (model.py:192). Its forward hands the
// resident logits on as a non-leaf alias, its backward receives d(logits)
// and hands nothing further, as a C++ node, as the matmul's own backward
// is, so a timed step carries no Python node of its own.
struct HeadOutput : public torch::autograd::Function<HeadOutput> {
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& logits,
                            const at::Tensor& anchor) {
    (void)ctx;
    (void)anchor;
    return logits.alias();
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    (void)ctx;
    (void)grads;
    return {at::Tensor(), at::Tensor()};
  }
};

at::Tensor head_output(const at::Tensor& logits, const at::Tensor& anchor) {
  return HeadOutput::apply(logits, anchor);
}

}  // namespace

PYBIND11_MODULE(_nmce_autograd, m) {
  m.doc() = "The one-pass loss at TP = 1 as a C++ autograd node over libnmce's C ABI.";
  m.def("one_pass_mean", &one_pass_mean, "mean one-pass loss (forward + backward in C++)");
  m.def("one_pass_mean_checked", &one_pass_mean_checked,
        "one_pass_mean after the target check; ValueError on a target outside the vocabulary");
  m.def("assumed_of", &assumed_of, "the assumed upstream value saved by a one-pass loss");
  m.def("set_timing", &set_timing, "time every launch with HIP events while on");
  m.def("take_timeline", &take_timeline, "(name, ms) of the launches timed since the last call");
  m.def("head_output", &head_output,
        "logits as a non-leaf alias through a C++ node whose backward hands nothing on "
        "(stands for the LM-head matmul in measurements)");
}
