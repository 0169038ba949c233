// C-ABI glue shared by all entry points: per-thread error text and the ABI version.
#include "exl3_common.h"

namespace exl3 {

std::string& last_error()
{
    static thread_local std::string msg;
    return msg;
}

}  // namespace exl3

extern "C" const char* exl3_last_error(void) { return exl3::last_error().c_str(); }

extern "C" int exl3_abi_version(void) { return 10; }
