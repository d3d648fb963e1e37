// Quality certificates of the approximate modes.  "<weights>.hip.cert" holds the header line SHIELDV_HIP_CERT_V2,
// then one line per certified (weights, mode, compute revision):
//   "<weights sha256> <mode> <revision> PASS <cert json> <cert json sha256> threshold=<%.17g>"
// A mode loads only if such a line names this SHA-256, this mode and this library's revision, and its threshold
// is exactly the sidecar's (the reference's rule: engine/include/shv_cuda.h:17-26).
#include "cert.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <vector>

namespace shv {

namespace {
std::vector<std::string> fields_of(const std::string& line) {
    std::vector<std::string> out;
    std::istringstream in(line);
    for (std::string f; in >> f;) out.push_back(f);
    return out;
}

// "threshold=<double>" with nothing after the number, else NaN
double threshold_field(const std::vector<std::string>& f) {
    static const std::string key = "threshold=";
    for (size_t i = 4; i < f.size(); ++i) {
        if (f[i].compare(0, key.size(), key) != 0) continue;
        const char* s = f[i].c_str() + key.size();
        char* end = nullptr;
        const double v = std::strtod(s, &end);
        return (end != s && *end == '\0') ? v : std::nan("");
    }
    return std::nan("");
}
}  // namespace

std::string certificate_problem(const std::string& weights, const std::string& sha, const std::string& mode,
                                double threshold, const std::string& revision) {
    const std::string path = weights + ".hip.cert";
    std::ifstream in(path);
    if (!in) return "mode " + mode + " is uncertified: no certificate file at " + path;
    std::vector<std::string> lines;
    for (std::string l; std::getline(in, l);) lines.push_back(l);
    if (lines.empty()) return "certificate file " + path + " is empty";
    std::string head = lines[0];
    head.erase(head.find_last_not_of(" \r\t") + 1);
    if (head != "SHIELDV_HIP_CERT_V2") return "certificate file " + path + " lacks the SHIELDV_HIP_CERT_V2 header line";

    bool named = false;
    double named_threshold = std::nan("");
    for (size_t i = 1; i < lines.size(); ++i) {
        const std::vector<std::string> f = fields_of(lines[i]);
        if (f.size() < 4 || f[0] != sha || f[1] != mode || f[2] != revision || f[3] != "PASS") continue;
        const double t = threshold_field(f);
        if (std::isfinite(t) && t == threshold) return "";
        named = true;
        named_threshold = t;
    }
    if (named) {
        char nums[160];
        std::snprintf(nums, sizeof nums, "certified for threshold %.17g, the sidecar sets %.17g", named_threshold,
                      threshold);
        return "mode " + mode + " is uncertified at this threshold: certificate file " + path + " " + nums + " (" +
               weights + ".json)";
    }
    return "mode " + mode + " is uncertified: certificate file " + path + " has no PASS line for weights " + sha +
           " at revision " + revision;
}

}  // namespace shv
