// The kernel variant each launcher chose, for plan recording: every launcher
// in the *.hip files calls note_launch() after it launches, and the decoders
// read last_launch() to record (operation, kernel, batch) steps -- the
// reference's PlanIR step (src/fortai_plan_ir.f90:7-21).
#include "fortai_hip_kernels.h"

#include <cstdarg>
#include <cstdio>

namespace fortai_hip {

namespace {
thread_local char g_last[256] = "";
}

void note_launch(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last, sizeof(g_last), fmt, ap);
    va_end(ap);
}

const char *last_launch() { return g_last; }

const char *prologue_name(Prologue p) {
    switch (p) {
    case Prologue::Q8: return "q8";
    case Prologue::F32: return "f32";
    case Prologue::RMSNORM: return "rmsnorm";
    case Prologue::Q8L: return "q8l";
    case Prologue::GATED: return "gated";
    }
    return "?";
}

const char *epilogue_name(Epilogue e) {
    switch (e) {
    case Epilogue::STORE: return "store";
    case Epilogue::ADD: return "add";
    case Epilogue::SILU_PAIR: return "silu_pair";
    }
    return "?";
}

}  // namespace fortai_hip
