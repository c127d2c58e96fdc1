/*
 * g4s_runtime.h -- host-side helpers shared by the library's entry points.
 */
#ifndef G4S_RUNTIME_H
#define G4S_RUNTIME_H

namespace g4s {

/* The message g4s_last_error(NULL) returns on this thread: the last failed
 * g4s_create or handle-free entry point.  set_ returns `code`. */
int set_null_handle_error(int code, const char* fmt, ...);
void clear_null_handle_error();

}  // namespace g4s

#endif
