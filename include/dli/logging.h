#pragma once

// Leveled logging with a replaceable sink. API as include/dli/logging.h:12-44 of the
// reference, with one change: the LOG_* macros test the level before a message is built,
// so a dropped message costs one relaxed atomic load instead of a string format.

#include <atomic>
#include <functional>
#include <iosfwd>
#include <ostream>
#include <sstream>
#include <string>
#include <string_view>

namespace dli {

enum class LogSeverity { Debug, Info, Warn, Error };

using LogSink = std::function<void(LogSeverity severity, std::string_view file, int line,
                                   std::string_view message)>;

const char* toString(LogSeverity severity);
void setLogLevel(LogSeverity severity);
LogSeverity logLevel();
void setLogSink(LogSink sink);
void resetLogSink();

namespace detail {
extern std::atomic<int> g_log_threshold;
inline bool logEnabled(LogSeverity severity) {
  return static_cast<int>(severity) >= g_log_threshold.load(std::memory_order_relaxed);
}
// Swallows the stream expression so the macro below is a single void expression.
struct LogVoidify {
  void operator&(std::ostream&) {}
};
}  // namespace detail

class LogMessage {
 public:
  LogMessage(LogSeverity severity, const char* file, int line);
  LogMessage(const LogMessage&) = delete;
  LogMessage& operator=(const LogMessage&) = delete;
  ~LogMessage() noexcept;

  std::ostream& stream() { return stream_; }

 private:
  LogSeverity severity_;
  const char* file_;
  int line_;
  std::ostringstream stream_;
};

}  // namespace dli

#define DLI_LOG_AT(sev)                                    \
  !::dli::detail::logEnabled(sev) ? (void)0                \
                                  : ::dli::detail::LogVoidify() & \
                                        ::dli::LogMessage(sev, __FILE__, __LINE__).stream()

#define LOG_DEBUG DLI_LOG_AT(::dli::LogSeverity::Debug)
#define LOG_INFO DLI_LOG_AT(::dli::LogSeverity::Info)
#define LOG_WARN DLI_LOG_AT(::dli::LogSeverity::Warn)
#define LOG_ERROR DLI_LOG_AT(::dli::LogSeverity::Error)
