// Functions shared between librq's translation units; hidden, not part of the
// C-ABI.
#ifndef RQ_INTERNAL_H
#define RQ_INTERNAL_H

#include <string>

#include "../../include/rq.h"

// Sets the calling thread's rq_last_error() message and returns `code`.
__attribute__((visibility("hidden"))) rq_status rq_fail_msg(rq_status code, const std::string& msg);

#endif
