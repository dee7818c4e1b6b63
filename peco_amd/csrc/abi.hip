// Status strings for the C-ABI (peco/kernels/kmeans.cu:220, sparse_attention.cu:232).
// 0 is success, hipError_t values pass through, PECO-specific codes start at 20001.
#include "common.hpp"

using namespace peco;

namespace {
const char* peco_status(int code) {
    switch (code) {
        case kWorkspaceTooSmall: return "PECO: workspace too small";
        case kUnsupportedShape: return "PECO: unsupported shape (head dim must be 64 or 128; cluster counts within limits)";
        case kUnsupportedDtype: return "PECO: unsupported dtype";
        case kScratchExceeded:
            return "PECO: problem exceeds the static scratch of peco_sparse_attention_noalloc "
                   "(work list of at most 1048576 int32; use peco_sparse_attention with a workspace)";
        default: return hipGetErrorString(static_cast<hipError_t>(code));
    }
}
}  // namespace

PECO_API const char* peco_cluster_error_message(int code) { return peco_status(code); }

PECO_API const char* peco_attention_error_string(int code) { return peco_status(code); }

PECO_API int peco_abi_version(void) { return 5; }
