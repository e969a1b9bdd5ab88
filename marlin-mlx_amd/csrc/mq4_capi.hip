// Library-wide C-ABI entry points of libmq4 (error reporting, version).
#include "mq4_host.h"

namespace mq4 {
std::string& last_error_ref() {
    thread_local std::string msg;
    return msg;
}
}  // namespace mq4

extern "C" const char* mq4_last_error(void) { return mq4::last_error_ref().c_str(); }

extern "C" int mq4_version(void) { return 100; }  // 0.1.0
