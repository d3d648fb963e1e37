// TEST INFRASTRUCTURE ONLY: a C entry point into the reference SHIELD-A engine's sequence stages, compiled together
// with that engine's own sources (oracle/Makefile, target ref).  It loads SHLDA001 weights with the reference's
// loader (engine/audio/weights.cpp), checks the sequence tensors (engine/audio/sequence.cpp:304-331) and evaluates
// shield::sequence (sequence.cpp:346: 125 tokens + readout -> GDN-A -> GDN-B x2 -> SISA last row -> head -> logit)
// in the engine's default exact mode.  With a dump directory, the engine writes its stage tensors there
// (SHIELD_DUMP_DIR, sequence.cpp:36-41).
#include "core.hpp"

#include <cstdlib>
#include <cstring>
#include <exception>
#include <string>

namespace {
thread_local std::string g_err;
}

extern "C" {

__attribute__((visibility("default"))) void* ora_audio_load(const char* path) {
    try {
        auto* w = new shield::Weights(path);
        try {
            shield::validate_sequence_weights(*w);
        } catch (...) {
            delete w;
            throw;
        }
        return w;
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

__attribute__((visibility("default"))) const char* ora_audio_error() { return g_err.c_str(); }

__attribute__((visibility("default"))) int ora_audio_sequence(void* h, const float* tokens, float* logit,
                                                              const char* dump_dir) {
    try {
        if (dump_dir && *dump_dir) setenv("SHIELD_DUMP_DIR", dump_dir, 1);
        shield::sequence(*static_cast<shield::Weights*>(h), tokens, *logit);
        if (dump_dir && *dump_dir) unsetenv("SHIELD_DUMP_DIR");
        return 0;
    } catch (const std::exception& e) {
        unsetenv("SHIELD_DUMP_DIR");
        g_err = e.what();
        return -1;
    }
}

__attribute__((visibility("default"))) void ora_audio_free(void* h) { delete static_cast<shield::Weights*>(h); }
}
