// Library-wide C entry points: error string and ABI version.
#include "pl_common.h"

extern "C" const char* pl_last_error(void) { return pl::error_buffer(); }

extern "C" int pl_version(void) { return (1 << 16) | 0; }
