// Library-internal helpers shared by the translation units of libemrs.
#ifndef EMRS_INTERNAL_H
#define EMRS_INTERNAL_H

#include <string>

namespace emrs_internal {
// Record `msg` as this thread's last error (read by emrs_last_error) and return `code`.
int fail(int code, const std::string &msg);
void clear_error();
}  // namespace emrs_internal

#endif
