// Host-side helpers shared by the translation units of libd8s_hip.so (not part of the C ABI).
#ifndef D8S_HOST_H
#define D8S_HOST_H

#include <string>

#define D8S_HIDDEN __attribute__((visibility("hidden")))

// Records `msg` as the calling thread's last error (d8s_last_error) and returns `code`.
D8S_HIDDEN int d8s_host_fail(int code, const std::string& msg);
// 0 if the last launch succeeded, else the HIP error (recorded as above, prefixed with `what`).
D8S_HIDDEN int d8s_host_launched(const char* what);
// Compute units of the current device.
D8S_HIDDEN int d8s_host_cu_count();

#endif
