// Minimal logging: VELOMIND_LOG(level, message-string) to a replaceable
// handler (stderr by default).  Avoids <format>, which this toolchain's
// libstdc++ lacks.
#pragma once

#include <string>

namespace velomind::internal {

enum class LogLevel { Debug, Info, Warn, Error };
using LogHandler = void (*)(LogLevel, const std::string&);

void set_log_handler(LogHandler handler);
void log_message(LogLevel level, const std::string& message);

}  // namespace velomind::internal

#define VELOMIND_LOG(LEVEL, MSG) ::velomind::internal::log_message(::velomind::internal::LogLevel::LEVEL, (MSG))
