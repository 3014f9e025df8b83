// Thread-local last-error message behind frn_last_error().
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "../common.hpp"

static thread_local std::string g_err;

frn_status frn_fail(frn_status st, const char* fmt, ...) {
  char buf[768];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return st;
}

extern "C" const char* frn_last_error(void) { return g_err.c_str(); }
