// TEST INFRASTRUCTURE ONLY: C entry points into the reference SHIELD-A engine (its sequence stages, its frontend and
// the two together), compiled together
// with that engine's own sources (oracle/Makefile, target ref).  It loads SHLDA001 weights with the reference's
// loader (engine/audio/weights.cpp), checks the sequence tensors (engine/audio/sequence.cpp:304-331) and evaluates
// shield::sequence (sequence.cpp:346: 125 tokens + readout -> GDN-A -> GDN-B x2 -> SISA last row -> head -> logit)
// in the engine's default exact mode.  With a dump directory, the engine writes its stage tensors there
// (SHIELD_DUMP_DIR, sequence.cpp:36-41).
#include "core.hpp"
#include "frontend.hpp"
#include "sequence_cache.hpp"

#include <cstdlib>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

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

// The frontend alone (shield::frontend_cnn, engine/audio/frontend.cpp:258-280, no cache): 160,000 PCM samples ->
// tokens [125][384].  With a dump directory the engine also writes mel.f32 ([80][997]) and cnn.f32 there.
__attribute__((visibility("default"))) int ora_audio_frontend(void* h, const float* pcm, float* tokens,
                                                              const char* dump_dir) {
    try {
        if (dump_dir && *dump_dir) setenv("SHIELD_DUMP_DIR", dump_dir, 1);
        std::vector<float> out;
        shield::frontend_cnn(*static_cast<shield::Weights*>(h), pcm, out, nullptr);
        if (dump_dir && *dump_dir) unsetenv("SHIELD_DUMP_DIR");
        if (out.size() != 125 * 384) throw std::runtime_error("frontend returned an unexpected token count");
        std::memcpy(tokens, out.data(), out.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        unsetenv("SHIELD_DUMP_DIR");
        g_err = e.what();
        return -1;
    }
}

// PCM -> logit as the engine's worker computes it (engine/audio/api.cpp:58-70 without a cache): frontend, then the
// sequence stages.
__attribute__((visibility("default"))) int ora_audio_predict(void* h, const float* pcm, float* logit) {
    try {
        std::vector<float> tokens;
        const auto& w = *static_cast<shield::Weights*>(h);
        shield::frontend_cnn(w, pcm, tokens, nullptr);
        shield::sequence(w, tokens.data(), *logit);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// Frees the weights after dropping the engine's caches keyed by their addresses (packed GEMM weights, prepared
// frontend tables, projected readouts), as the engine's own model free does (engine/audio/api.cpp:56-57): a later
// load may reuse the addresses.
__attribute__((visibility("default"))) void ora_audio_free(void* h) {
    auto* w = static_cast<shield::Weights*>(h);
    if (!w) return;
    shield::release_sequence_weights(*w);
    shield::release_frontend_weights(*w);
    shield::release_kernel_weights(*w);
    delete w;
}
}
