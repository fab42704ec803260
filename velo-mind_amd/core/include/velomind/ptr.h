// Pointer aliases used across the VeloMind API (include/velomind/ptr.h:3-7 in
// the reference): pX, ppX, pConstX, ppConstX for a type X.
#pragma once

#define VELOMIND_EXPORT_PTR(type)        \
    using p##type = type*;               \
    using pp##type = type**;             \
    using pConst##type = const type*;    \
    using ppConst##type = const type**;
