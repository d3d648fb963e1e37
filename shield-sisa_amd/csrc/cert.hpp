// Certificate check of the approximate modes (fp16 / bf16): see cert.cpp for the file format.
#pragma once
#include <string>

namespace shv {

// "" if "<weights>.hip.cert" certifies (sha, mode, revision) at exactly `threshold`, else the reason it does not.
std::string certificate_problem(const std::string& weights, const std::string& sha, const std::string& mode,
                                double threshold, const std::string& revision);

}  // namespace shv
