#pragma once

// Opt-in operator profiling of Engine::run, as designed in the reference's
// .codex/profiling_design.md (its proposed include/dli/profiler.h; not implemented there).
//
// For every graph node a session records the host time inside Operator::compute and, for nodes
// with a device input, the device time between two HIP events recorded on the run's stream
// before and after the node. Nothing waits for the device during a run: event pairs are
// resolved by finalize(). The session then writes one "dli.profile.v1" JSON document; durations
// and timestamps are integer nanoseconds. CPU and GPU times are kept apart and never summed.
//
// Lifecycle: runs (Engine::run with RunOptions{&session}) -> finalize() (waits for the last
// recorded event) -> report() / toJson() / writeJson(). Another run after finalize() throws
// std::logic_error, as does report() before it; a second finalize() does nothing. Events past
// max_events are dropped and counted; inference goes on. If events cannot be created (no
// device) the session keeps CPU timing and says so in its metadata. Device timing needs the
// nodes' work on the run's stream; it is not available while that stream is being captured
// into a HIP graph (such runs record CPU time only).

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

namespace dli {

struct Node;
class Tensor;

struct ProfileConfig {
  bool cpu = true;
  bool gpu = true;
  bool record_shapes = false;
  std::size_t max_events = 1'000'000;
};

struct ProfileRunRecord {
  std::int64_t run_id = 0;
  std::int64_t start_ns = 0;     // steady_clock, relative to the session's creation
  std::int64_t duration_ns = 0;  // host wall time of the whole Engine::run
  std::string status = "ok";     // "ok" or "error"
};

struct ProfileEventRecord {
  std::int64_t event_id = 0;
  std::int64_t run_id = 0;
  std::int64_t node_index = 0;
  std::string node_name;
  std::string op_type;
  std::uint64_t host_thread_id = 0;
  std::int64_t cpu_start_ns = 0;
  std::int64_t cpu_duration_ns = 0;
  std::int64_t gpu_duration_ns = -1;  // -1: not measured (host-only node, capture, no device)
  int device = -1;                    // device of the node's first device input, -1 for host
  std::uintptr_t stream = 0;
  std::string status = "ok";  // "ok" or "error" (compute threw)
  std::string shapes;         // with record_shapes: "in:[f32 2x3],... -> out:[...]"
};

struct ProfileReport {
  std::string created_utc;
  std::int64_t process_id = 0;
  bool gpu_timing = false;
  std::string gpu_error;  // why device timing is off, when it is
  bool record_shapes = false;
  std::int64_t dropped_events = 0;
  std::vector<ProfileRunRecord> runs;
  std::vector<ProfileEventRecord> events;
};

class ProfileSession {
 public:
  explicit ProfileSession(ProfileConfig config = {});
  ~ProfileSession();
  ProfileSession(const ProfileSession&) = delete;
  ProfileSession& operator=(const ProfileSession&) = delete;

  const ProfileConfig& config() const { return config_; }
  bool finalized() const { return finalized_; }

  void finalize();
  const ProfileReport& report() const;
  std::string toJson() const;
  void writeJson(const std::string& path) const;

  // Engine hooks. beginRun returns the run id; stream is the run's hipStream_t (nullptr = null
  // stream) and capturing says whether it is being captured into a graph.
  std::int64_t beginRun(void* stream, bool capturing);
  void endRun(std::int64_t run_id, bool ok);

  // One node's span: created before Operator::compute, finished after it (ok) or during
  // unwinding (error). Move-only.
  class Scope {
   public:
    Scope() = default;
    Scope(Scope&& other) noexcept;
    Scope& operator=(Scope&&) = delete;
    ~Scope();
    void finish(bool ok, const std::vector<Tensor*>* outputs);

   private:
    friend class ProfileSession;
    ProfileSession* session_ = nullptr;
    std::size_t slot_ = 0;
    std::int64_t cpu_start_ns_ = 0;
    bool done_ = true;
  };
  Scope beginOperator(std::int64_t run_id, std::int64_t node_index, const Node& node,
                      const std::vector<const Tensor*>& inputs);

 private:
  struct Pending {
    void* start = nullptr;
    void* stop = nullptr;
  };
  std::int64_t nowNs() const;
  void finishScope(Scope& scope, bool ok, const std::vector<Tensor*>* outputs);

  ProfileConfig config_;
  std::int64_t origin_ns_ = 0;
  mutable std::mutex mutex_;
  bool finalized_ = false;
  void* run_stream_ = nullptr;
  bool run_gpu_ = false;  // device timing for the current run
  ProfileReport report_;
  std::vector<Pending> pending_;  // per event (same index), device event pair or none
  std::vector<void*> free_events_;
  void* last_stop_ = nullptr;  // the last device event recorded (finalize waits for it)
};

// Options of one Engine::run. profiler: non-owning, valid through the run.
struct RunOptions {
  ProfileSession* profiler = nullptr;
};

}  // namespace dli
