// Matvec launches over several input rows (MvArgs::rows): batched decode rows
// of a few sequences read each weight once for all of them.
#include "matvec.h"

namespace ribn {
namespace {

// R input rows through one launch (MvArgs::rows)
template <int MODE>
hipError_t rows_dispatch(const MvArgs& a, int n_wg, hipStream_t st) {
    switch (a.rows) {
    case 2: return matvec_dispatch<MODE, 2>(a, n_wg, st);
    case 3: return matvec_dispatch<MODE, 3>(a, n_wg, st);
    case 4: return matvec_dispatch<MODE, 4>(a, n_wg, st);
    default: return hipErrorInvalidValue;
    }
}


}  // namespace

hipError_t launch_matvec_rows(const MvArgs& a, int n_wg, hipStream_t st) {
    switch (a.mode) {
    case MV_STORE: return rows_dispatch<MV_STORE>(a, n_wg, st);
    case MV_ADD: return rows_dispatch<MV_ADD>(a, n_wg, st);
    case MV_SILU: return rows_dispatch<MV_SILU>(a, n_wg, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ribn
