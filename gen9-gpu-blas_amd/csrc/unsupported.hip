// Entry points of the reference ABI that this build declares and exports but does not compute yet: the level-2
// symmetric/triangular/banded/packed functions (reference: lib/src/level12.c:267-519).
// Each one validates its type and arguments the way the reference does, then returns GEN9BLAS_ERR_UNSUPPORTED with a
// message, so a caller (the BLAS shim among them) falls back to its CPU path. Exporting them keeps the ABI whole:
// loaders that bind every symbol of the header (the ctypes module, the Rust crate) work unchanged.
#include "internal.h"

using namespace g9;

namespace {
int check_type(int type) {
    G9_TRY(begin());
    if (type < 0 || type > 3) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", type);
    return 0;
}
int not_built(const char *f) { G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "%s is not implemented in this build", f); }
}  // namespace

extern "C" {

#define G9_UNBUILT(name, ...)                 \
    int name(int type, __VA_ARGS__) {         \
        G9_TRY(check_type(type));             \
        return not_built(#name);              \
    }

G9_UNBUILT(gen9blas_symv, int, int, double, const void *, int, const void *, int, double, void *, int)
G9_UNBUILT(gen9blas_trmv, int, int, int, int, const void *, int, void *, int)
G9_UNBUILT(gen9blas_trsv, int, int, int, int, const void *, int, void *, int)
G9_UNBUILT(gen9blas_syr, int, int, double, const void *, int, void *, int)
G9_UNBUILT(gen9blas_syr2, int, int, double, const void *, int, const void *, int, void *, int)
G9_UNBUILT(gen9blas_gbmv, int, int, int, int, int, double, const void *, int, const void *, int, double, void *, int)
G9_UNBUILT(gen9blas_sbmv, int, int, int, double, const void *, int, const void *, int, double, void *, int)
G9_UNBUILT(gen9blas_tbmv, int, int, int, int, int, const void *, int, void *, int)
G9_UNBUILT(gen9blas_tbsv, int, int, int, int, int, const void *, int, void *, int)
G9_UNBUILT(gen9blas_spmv, int, int, double, const void *, const void *, int, double, void *, int)
G9_UNBUILT(gen9blas_tpmv, int, int, int, int, const void *, void *, int)
G9_UNBUILT(gen9blas_tpsv, int, int, int, int, const void *, void *, int)
G9_UNBUILT(gen9blas_spr, int, int, double, const void *, int, void *)
G9_UNBUILT(gen9blas_spr2, int, int, double, const void *, int, const void *, int, void *)

}  // extern "C"
