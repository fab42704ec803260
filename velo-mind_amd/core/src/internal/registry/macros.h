// Token pasting for the static-registration macros.
#pragma once
#define VELOMIND_CONCAT_INNER_(a, b) a##b
#define VELOMIND_CONCAT_(a, b) VELOMIND_CONCAT_INNER_(a, b)
