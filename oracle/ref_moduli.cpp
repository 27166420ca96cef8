// ref_moduli.cpp -- exports the REFERENCE's own CRT table builder, compiled from its unmodified
// header (src/moduli.h:124-181, self-contained C++) by `make -C oracle ref`, into
// oracle/_ref/libref_moduli.so.  Test infrastructure only: tests/test_oracle.py compares its table,
// byte for byte, with the oracle's restatement (oz2o_build_tables).  The header is included from
// where it lies under the reference checkout; nothing of it is copied here.
#include <cstddef>
#include <cstring>

#include "moduli.h"

extern "C" size_t ref_crt_tables_size() { return sizeof(oz2_crt_tables); }

// Builds the table into out (cap bytes); returns the builder's status, or -1 if out is too small.
extern "C" int ref_build_crt_tables(void* out, size_t cap) {
  if (cap < sizeof(oz2_crt_tables)) return -1;
  oz2_crt_tables t;
  std::memset(&t, 0, sizeof t);
  const int rc = oz2_build_crt_tables(&t);
  std::memcpy(out, &t, sizeof t);
  return rc;
}
