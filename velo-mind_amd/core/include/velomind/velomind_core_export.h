// Symbol visibility for libvelomind.so (this build's own export macro).
#pragma once
#define VELOMIND_CORE_EXPORT __attribute__((visibility("default")))
