// Leveled logging (reference behaviour: src/logging.cc:20-91 — default level WARN, a sink
// that receives severity/file/line/message, stderr when no sink is set).
#include "dli/logging.h"

#include <iostream>
#include <mutex>
#include <utility>

namespace dli {
namespace detail {
std::atomic<int> g_log_threshold{static_cast<int>(LogSeverity::Warn)};
}  // namespace detail

namespace {

struct SinkState {
  std::mutex mutex;
  LogSink sink;
};

SinkState& sinkState() {
  static SinkState* state = new SinkState;  // never destroyed: usable during static teardown
  return *state;
}

}  // namespace

const char* toString(LogSeverity severity) {
  static const char* const kNames[] = {"DEBUG", "INFO", "WARN", "ERROR"};
  const int index = static_cast<int>(severity);
  return (index >= 0 && index < 4) ? kNames[index] : "UNKNOWN";
}

void setLogLevel(LogSeverity severity) {
  detail::g_log_threshold.store(static_cast<int>(severity), std::memory_order_relaxed);
}

LogSeverity logLevel() {
  return static_cast<LogSeverity>(detail::g_log_threshold.load(std::memory_order_relaxed));
}

void setLogSink(LogSink sink) {
  auto& state = sinkState();
  std::lock_guard<std::mutex> lock(state.mutex);
  state.sink = std::move(sink);
}

void resetLogSink() { setLogSink(nullptr); }

LogMessage::LogMessage(LogSeverity severity, const char* file, int line)
    : severity_(severity), file_(file), line_(line) {}

LogMessage::~LogMessage() noexcept {
  try {
    if (!detail::logEnabled(severity_)) return;
    const std::string text = stream_.str();
    auto& state = sinkState();
    std::lock_guard<std::mutex> lock(state.mutex);
    if (state.sink) {
      state.sink(severity_, file_, line_, text);
    } else {
      std::cerr << '[' << toString(severity_) << "] " << file_ << ':' << line_ << ' ' << text
                << '\n';
    }
  } catch (...) {
    // A destructor must not throw; a failing sink drops the message.
  }
}

}  // namespace dli
