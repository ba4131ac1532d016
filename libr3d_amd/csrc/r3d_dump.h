/* r3d_dump.h -- env-gated launch capture (R3D_DUMP); see r3d_dump.cpp for the format. */
#ifndef R3D_DUMP_H
#define R3D_DUMP_H

#include "rad_abi.h"

namespace r3d {

/* true when R3D_DUMP is set and `row` matches R3D_DUMP_OPS (read once per process) */
bool dump_wanted(const char* row);
/* the pre-launch state of a wanted row's launch, or null once the row's R3D_DUMP_MAX
 * captures are taken; synchronises `s` */
void* dump_begin(const char* row, const RadArgs* a, RadStream s);
/* the post-launch state (synchronises `s`) and the capture's files; frees the handle */
void dump_end(void* handle, const RadArgs* a, RadStream s, int rc);

/* Run `impl(a, s)` as row `row`, captured when the environment asks for it. */
template <typename F>
inline int dump_wrap(const char* row, const RadArgs* a, RadStream s, F impl) {
    if (!dump_wanted(row)) return impl(a, s);
    void* h = dump_begin(row, a, s);
    const int rc = impl(a, s);
    dump_end(h, a, s, rc);
    return rc;
}

}  // namespace r3d

#endif /* R3D_DUMP_H */
