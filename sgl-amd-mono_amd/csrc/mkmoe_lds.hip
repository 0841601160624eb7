// LDS budget of the persistent launch, per compiled shape: the bytes of each stage's member of
// the LDS union (router, routing, gate_up, down), the part the down stage's members take, and
// the step's union of experts that lives beside them from the routing to the end. A host
// program (no GPU call): python sgl-amd-mono_amd/build.py --lds compiles and runs it.
#define MKMOE_UNIT 100  // the kernel source's definitions alone: no shape's kernels, no host code
#include "mkmoe_kernels.hip"

namespace {

template <class C>
void row(const char* name) {
  using namespace mkmoe;
  using D = DownSmem<C>;
  using G = GuSmem<C>;
  const size_t un = sizeof(Union<C>), st = sizeof(StageSmem<C>);
  printf("| %s | %d / %d / %d | %zu | %zu | %zu | %zu | %zu | %zu | %zu | %zu | %zu | %zu |\n", name, C::H, C::I,
         C::TMAX, sizeof(RouterSmem<C>), sizeof(RouteSmem<C>), sizeof(G), sizeof(G::m.wslot), sizeof(D),
         sizeof(D::wslot), sizeof(D::contrib), sizeof(D::shv), un, un + st);
}

}  // namespace

int main() {
  printf("| shape | H / I / tile rows | router | routing | gate_up | its weight slots | down | its weight slots "
         "| pick contributions | shared results | union of experts | launch total |\n");
  printf("|---|---|---|---|---|---|---|---|---|---|---|---|\n");
  row<mkmoe::CfgPlumbing>("plumbing FP8");
  row<mkmoe::CfgTp4Fp8>("TP4 FP8 (cfg 2)");
  row<mkmoe::CfgTp4Fp4>("TP4 MXFP4 row-major");
  row<mkmoe::CfgTp4Fp4Aiter>("TP4 MXFP4 shuffled (cfg 3, 4)");
  row<mkmoe::CfgTp2Fp4Norm>("TP2 MXFP4 + norm row-major");
  row<mkmoe::CfgTp2Fp4NormAiter>("TP2 MXFP4 + norm shuffled (cfg 5)");
  row<mkmoe::CfgV41Tp4>("V4.1 TP4");
  row<mkmoe::CfgV41Tp2>("V4.1 TP2");
  return 0;
}
