// Operator profiling session (design: .codex/profiling_design.md of the reference; the reference
// has no implementation). Device timing uses HIP events through the device C ABI (dli_hip.h).
#include "dli/profiler.h"

#include <unistd.h>

#include <chrono>
#include <cstdio>
#include <ctime>
#include <fstream>
#include <functional>
#include <sstream>
#include <stdexcept>
#include <thread>

#include "dli/graph.h"
#include "dli/tensor.h"
#include "dli/utils.h"
#include "dli_hip.h"

namespace dli {
namespace {

std::int64_t steadyNs() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

std::string utcNow() {
  const std::time_t t = std::time(nullptr);
  std::tm tm{};
  gmtime_r(&t, &tm);
  char buf[32];
  std::strftime(buf, sizeof(buf), "%Y-%m-%dT%H:%M:%SZ", &tm);
  return buf;
}

std::string jsonEscape(const std::string& s) {
  std::string out;
  out.reserve(s.size() + 2);
  for (const char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (static_cast<unsigned char>(c) < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", static_cast<unsigned>(c));
          out += buf;
        } else {
          out += c;
        }
    }
  }
  return out;
}

std::string describe(const Tensor& t) {
  std::ostringstream os;
  os << toString(t.dtype()) << ' ' << (t.isCuda() ? "cuda" : "cpu") << ' '
     << formatShape(t.shape());
  return os.str();
}

const Tensor* firstDeviceTensor(const std::vector<const Tensor*>& inputs) {
  for (const Tensor* t : inputs)
    if (t != nullptr && t->defined() && t->isCuda()) return t;
  return nullptr;
}

}  // namespace

ProfileSession::ProfileSession(ProfileConfig config) : config_(config), origin_ns_(steadyNs()) {
  report_.created_utc = utcNow();
  report_.process_id = static_cast<std::int64_t>(::getpid());
  report_.record_shapes = config_.record_shapes;
  report_.gpu_timing = config_.gpu;
  if (config_.gpu && dli_hip_available() == 0) {
    report_.gpu_timing = false;
    const char* why = dli_hip_load_error();
    report_.gpu_error = why != nullptr && *why != '\0' ? why : "no HIP device";
  }
}

ProfileSession::~ProfileSession() {
  // Releases device events; never writes files or throws.
  for (Pending& p : pending_) {
    if (p.start != nullptr) dli_hip_event_destroy(p.start);
    if (p.stop != nullptr) dli_hip_event_destroy(p.stop);
  }
  for (void* e : free_events_) dli_hip_event_destroy(e);
}

std::int64_t ProfileSession::nowNs() const { return steadyNs() - origin_ns_; }

std::int64_t ProfileSession::beginRun(void* stream, bool capturing) {
  std::lock_guard<std::mutex> lock(mutex_);
  if (finalized_) throw std::logic_error("ProfileSession: run after finalize()");
  ProfileRunRecord run;
  run.run_id = static_cast<std::int64_t>(report_.runs.size());
  run.start_ns = nowNs();
  report_.runs.push_back(run);
  run_stream_ = stream;
  run_gpu_ = report_.gpu_timing && !capturing;
  return run.run_id;
}

void ProfileSession::endRun(std::int64_t run_id, bool ok) {
  std::lock_guard<std::mutex> lock(mutex_);
  if (run_id < 0 || run_id >= static_cast<std::int64_t>(report_.runs.size())) return;
  ProfileRunRecord& run = report_.runs[static_cast<std::size_t>(run_id)];
  run.duration_ns = nowNs() - run.start_ns;
  run.status = ok ? "ok" : "error";
}

ProfileSession::Scope ProfileSession::beginOperator(std::int64_t run_id, std::int64_t node_index,
                                                    const Node& node,
                                                    const std::vector<const Tensor*>& inputs) {
  Scope scope;
  std::lock_guard<std::mutex> lock(mutex_);
  if (finalized_) throw std::logic_error("ProfileSession: run after finalize()");
  if (report_.events.size() >= config_.max_events) {
    ++report_.dropped_events;
    return scope;  // done_: nothing recorded for this node
  }
  ProfileEventRecord ev;
  ev.event_id = static_cast<std::int64_t>(report_.events.size());
  ev.run_id = run_id;
  ev.node_index = node_index;
  ev.node_name = node.name;
  ev.op_type = node.op_type;
  ev.host_thread_id = static_cast<std::uint64_t>(std::hash<std::thread::id>{}(std::this_thread::get_id()));
  ev.stream = reinterpret_cast<std::uintptr_t>(run_stream_);
  if (config_.record_shapes) {
    std::string s = "in:[";
    for (std::size_t i = 0; i < inputs.size(); ++i) {
      if (i) s += ", ";
      s += inputs[i] != nullptr && inputs[i]->defined() ? describe(*inputs[i]) : "none";
    }
    ev.shapes = s + "]";
  }
  Pending pending;
  if (const Tensor* dev = firstDeviceTensor(inputs)) {
    ev.device = dev->deviceId();
    if (run_gpu_) {
      auto take = [&]() -> void* {
        if (!free_events_.empty()) {
          void* e = free_events_.back();
          free_events_.pop_back();
          return e;
        }
        void* e = nullptr;
        return dli_hip_event_create(&e) == 0 ? e : nullptr;
      };
      pending.start = take();
      pending.stop = take();
      if (pending.start == nullptr || pending.stop == nullptr ||
          dli_hip_event_record(pending.start, run_stream_) != 0) {
        if (pending.start != nullptr) free_events_.push_back(pending.start);
        if (pending.stop != nullptr) free_events_.push_back(pending.stop);
        pending = Pending{};
      }
    }
  }
  report_.events.push_back(std::move(ev));
  pending_.push_back(pending);
  scope.session_ = this;
  scope.slot_ = report_.events.size() - 1;
  scope.done_ = false;
  scope.cpu_start_ns_ = nowNs();  // last, so the bookkeeping above is not charged to compute
  return scope;
}

void ProfileSession::finishScope(Scope& scope, bool ok, const std::vector<Tensor*>* outputs) {
  const std::int64_t end = nowNs();
  std::lock_guard<std::mutex> lock(mutex_);
  ProfileEventRecord& ev = report_.events[scope.slot_];
  Pending& pending = pending_[scope.slot_];
  if (config_.cpu) {
    ev.cpu_start_ns = scope.cpu_start_ns_;
    ev.cpu_duration_ns = end - scope.cpu_start_ns_;
  }
  ev.status = ok ? "ok" : "error";
  if (pending.start != nullptr) {
    if (ok && dli_hip_event_record(pending.stop, run_stream_) == 0) {
      last_stop_ = pending.stop;
    } else {  // a failed node has no device duration
      free_events_.push_back(pending.start);
      free_events_.push_back(pending.stop);
      pending = Pending{};
    }
  }
  if (config_.record_shapes && outputs != nullptr) {
    std::string s = " -> out:[";
    for (std::size_t i = 0; i < outputs->size(); ++i) {
      if (i) s += ", ";
      const Tensor* t = (*outputs)[i];
      s += t != nullptr && t->defined() ? describe(*t) : "none";
    }
    ev.shapes += s + "]";
  }
}

ProfileSession::Scope::Scope(Scope&& other) noexcept
    : session_(other.session_), slot_(other.slot_), cpu_start_ns_(other.cpu_start_ns_),
      done_(other.done_) {
  other.done_ = true;
}

ProfileSession::Scope::~Scope() {
  if (!done_ && session_ != nullptr) {
    done_ = true;
    try {
      session_->finishScope(*this, false, nullptr);  // unwinding: the node threw
    } catch (...) {
    }
  }
}

void ProfileSession::Scope::finish(bool ok, const std::vector<Tensor*>* outputs) {
  if (done_ || session_ == nullptr) return;
  done_ = true;
  session_->finishScope(*this, ok, outputs);
}

void ProfileSession::finalize() {
  std::lock_guard<std::mutex> lock(mutex_);
  if (finalized_) return;
  if (last_stop_ != nullptr && dli_hip_event_synchronize(last_stop_) != 0) {
    report_.gpu_error = std::string("waiting for the last event failed: ") + dli_hip_last_error();
  }
  for (std::size_t i = 0; i < pending_.size(); ++i) {
    Pending& p = pending_[i];
    if (p.start == nullptr) continue;
    float ms = 0.f;
    if (dli_hip_event_elapsed_ms(p.start, p.stop, &ms) == 0)
      report_.events[i].gpu_duration_ns = static_cast<std::int64_t>(ms * 1e6 + 0.5);
    free_events_.push_back(p.start);
    free_events_.push_back(p.stop);
    p = Pending{};
  }
  for (void* e : free_events_) dli_hip_event_destroy(e);
  free_events_.clear();
  last_stop_ = nullptr;
  finalized_ = true;
}

const ProfileReport& ProfileSession::report() const {
  if (!finalized_) throw std::logic_error("ProfileSession: report() before finalize()");
  return report_;
}

std::string ProfileSession::toJson() const {
  const ProfileReport& r = report();
  std::ostringstream os;
  os << "{\n  \"schema\": \"dli.profile.v1\",\n  \"clock\": \"steady_clock\",\n"
     << "  \"metadata\": {\"created_utc\": \"" << r.created_utc << "\", \"process_id\": "
     << r.process_id << ", \"runtime\": \"dl-inference gfx950\", \"gpu_timing\": "
     << (r.gpu_timing ? "true" : "false") << ", \"gpu_timing_api\": \"hip_events\", "
     << "\"record_shapes\": " << (r.record_shapes ? "true" : "false")
     << ", \"dropped_events\": " << r.dropped_events;
  if (!r.gpu_error.empty()) os << ", \"gpu_error\": \"" << jsonEscape(r.gpu_error) << "\"";
  os << "},\n  \"runs\": [";
  for (std::size_t i = 0; i < r.runs.size(); ++i) {
    const ProfileRunRecord& run = r.runs[i];
    os << (i ? ",\n    " : "\n    ") << "{\"run_id\": " << run.run_id << ", \"start_ns\": "
       << run.start_ns << ", \"duration_ns\": " << run.duration_ns << ", \"status\": \""
       << run.status << "\"}";
  }
  os << (r.runs.empty() ? "]" : "\n  ]") << ",\n  \"events\": [";
  for (std::size_t i = 0; i < r.events.size(); ++i) {
    const ProfileEventRecord& e = r.events[i];
    os << (i ? ",\n    " : "\n    ") << "{\"event_id\": " << e.event_id
       << ", \"run_id\": " << e.run_id << ", \"parent_id\": null, \"category\": \"graph_operator\""
       << ", \"node_index\": " << e.node_index << ", \"node_name\": \"" << jsonEscape(e.node_name)
       << "\", \"op_type\": \"" << jsonEscape(e.op_type) << "\", \"host_thread_id\": "
       << e.host_thread_id << ", \"cpu_start_ns\": " << e.cpu_start_ns
       << ", \"cpu_duration_ns\": " << e.cpu_duration_ns << ", \"gpu_duration_ns\": ";
    if (e.gpu_duration_ns >= 0)
      os << e.gpu_duration_ns;
    else
      os << "null";
    os << ", \"device\": " << e.device << ", \"stream\": \"0x" << std::hex << e.stream << std::dec
       << "\", \"status\": \"" << e.status << "\"";
    if (!e.shapes.empty()) os << ", \"shapes\": \"" << jsonEscape(e.shapes) << "\"";
    os << "}";
  }
  os << (r.events.empty() ? "]" : "\n  ]") << "\n}\n";
  return os.str();
}

void ProfileSession::writeJson(const std::string& path) const {
  const std::string text = toJson();
  std::ofstream out(path);
  if (!out) throw std::runtime_error("ProfileSession: cannot open " + path);
  out << text;
  if (!out) throw std::runtime_error("ProfileSession: write failed: " + path);
}

}  // namespace dli
