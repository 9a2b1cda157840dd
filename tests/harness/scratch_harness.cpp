// Test harness: the scratch ownership rules (scratch_registry.h) over fake
// runtime operations that log every call, so the rules are checked without a
// GPU.  Test infrastructure only; built into tests/harness/libscratch_harness.so.
#include <stdio.h>
#include <string.h>

#include <string>

#include "scratch_registry.h"

namespace {

std::string g_log;   // one line per runtime call
int g_device = 0;
int g_fail_alloc = 0;
long g_next = 0x1000;

void logf(const char* op, long a, long b) {
    char buf[96];
    snprintf(buf, sizeof(buf), "%s %ld %ld\n", op, a, b);
    g_log += buf;
}

int fake_device(int* d) {
    *d = g_device;
    return 0;
}
int fake_allocate(void** p, size_t bytes) {
    if (g_fail_alloc) return 2;   // hipErrorOutOfMemory
    *p = (void*)g_next;
    logf("alloc", g_next, (long)bytes);
    g_next += 0x1000;
    return 0;
}
int fake_zero(void* p, size_t bytes, void* stream) {
    logf("zero", (long)p, (long)stream);
    (void)bytes;
    return 0;
}
int fake_sync(void* stream) {
    logf("sync", (long)stream, 0);
    return 0;
}
int fake_release(void* p) {
    logf("free", (long)p, 0);
    return 0;
}

s2::ScratchRegistry* g_reg = 0;

}  // namespace

extern "C" {

void hs_reset() {
    delete g_reg;
    const s2::ScratchOps ops = {fake_device, fake_allocate, fake_zero, fake_sync, fake_release};
    g_reg = new s2::ScratchRegistry(ops);
    g_log.clear();
    g_device = 0;
    g_fail_alloc = 0;
    g_next = 0x1000;
}
void hs_set_device(int d) { g_device = d; }
void hs_fail_alloc(int f) { g_fail_alloc = f; }
int hs_acquire(int kind, long stream, long bytes) { return g_reg->acquire(kind, (void*)stream, (size_t)bytes); }
int hs_release(int kind, long stream) { return g_reg->release(kind, (void*)stream); }
int hs_get(int kind, long stream, long bytes, long* out) {
    void* p = 0;
    const int ret = g_reg->get(kind, (void*)stream, (size_t)bytes, &p);
    *out = (long)p;
    return ret;
}
int hs_owners(int kind, long stream) { return g_reg->owners(kind, (void*)stream); }
// Copies the call log (and clears it); returns its length.
int hs_take_log(char* buf, int cap) {
    const int n = (int)g_log.size();
    if (buf && cap > 0) {
        strncpy(buf, g_log.c_str(), (size_t)cap - 1);
        buf[cap - 1] = 0;
    }
    g_log.clear();
    return n;
}

}  // extern "C"
