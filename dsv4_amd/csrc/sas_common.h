// Internal helpers shared by the libsas translation units.
#pragma once

#include <cstdarg>
#include <cstdio>
#include <string>

namespace sas {

// Record a formatted error message for sas_last_error() and return `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

}  // namespace sas
