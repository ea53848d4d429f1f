// Runs the second-order uDTW sweeps of torchwarp_amd/csrc/udtw_tangent.hip
// on the CPU: the very function the kernel calls (tangent_pair), for one
// pair at a time, with a workgroup of CPU threads meeting at a barrier where
// the kernel has its workgroup barrier. Built under AddressSanitizer by
// tests/test_tangent_host.py, which compares the outputs with the oracle.
//
// usage: tangent_host B N M has_penalty gamma bandwidth threads in.bin out.bin
//   in.bin:  cost, pen, t_cost, t_pen [B,N,M]; grad_r, grad_p, t_grad_r,
//            t_grad_p [B] (float64; the penalty arrays only if has_penalty)
//   out.bin: t_d_cost [B,N,M], t_d_pen [B,N,M] (if has_penalty), t_r [B],
//            t_p [B] (if has_penalty)
#include "../../torchwarp_amd/csrc/udtw_tangent.hip"

#include <pthread.h>

#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

namespace tw {
namespace {
struct HostWorkgroup {
  int t, n;
  pthread_barrier_t* bar;
  int tid() const { return t; }
  int size() const { return n; }
  void sync() const { pthread_barrier_wait(bar); }
};
}  // namespace
}  // namespace tw

int main(int argc, char** argv) {
  if (argc != 10) return 2;
  const int B = atoi(argv[1]), N = atoi(argv[2]), M = atoi(argv[3]), pen = atoi(argv[4]);
  const double gamma = atof(argv[5]), band = atof(argv[6]);
  const int threads = atoi(argv[7]);
  const size_t nm = (size_t)N * M, bnm = (size_t)B * nm;
  FILE* f = fopen(argv[8], "rb");
  if (!f) return 3;
  // exactly sized heap arrays, so that the sanitizer sees every overrun
  auto read = [&](size_t n) {
    double* p = new double[n];
    if (fread(p, sizeof(double), n, f) != n) exit(4);
    return p;
  };
  double* C = read(bnm);
  double* Q = pen ? read(bnm) : nullptr;
  double* TC = read(bnm);
  double* TQ = pen ? read(bnm) : nullptr;
  double* gr = read(B);
  double* gp = pen ? read(B) : nullptr;
  double* tgr = read(B);
  double* tgp = pen ? read(B) : nullptr;
  fclose(f);
  double* oc = new double[bnm];
  double* oq = pen ? new double[bnm] : nullptr;
  double* orr = new double[B];
  double* op = pen ? new double[B] : nullptr;
  double* planes = new double[(size_t)B * tw::plane_elems(N, M, pen)];
  tw::TanArgs<double> a;
  a.cost = C;
  a.pen = Q;
  a.tcost = TC;
  a.tpen = TQ;
  a.gr = gr;
  a.gp = gp;
  a.tgr = tgr;
  a.tgp = tgp;
  a.out_c = oc;
  a.out_q = oq;
  a.out_r = orr;
  a.out_p = op;
  a.planes = planes;
  a.gring = nullptr;
  a.ring = (long long)tw::ring_elems(N, pen);
  a.N = N;
  a.M = M;
  a.gamma = gamma;
  a.band = band;
  for (int b = 0; b < B; ++b) {
    double* ring = new double[a.ring];
    pthread_barrier_t bar;
    pthread_barrier_init(&bar, nullptr, threads);
    std::vector<std::thread> team;
    for (int t = 0; t < threads; ++t) {
      team.emplace_back([&, t] {
        const tw::HostWorkgroup wg{t, threads, &bar};
        if (pen) {
          tw::tangent_pair<double, true>(a, b, ring, wg);
        } else {
          tw::tangent_pair<double, false>(a, b, ring, wg);
        }
      });
    }
    for (auto& th : team) th.join();
    pthread_barrier_destroy(&bar);
    delete[] ring;
  }
  f = fopen(argv[9], "wb");
  if (!f) return 5;
  fwrite(oc, sizeof(double), bnm, f);
  if (pen) fwrite(oq, sizeof(double), bnm, f);
  fwrite(orr, sizeof(double), B, f);
  if (pen) fwrite(op, sizeof(double), B, f);
  fclose(f);
  for (double* p : {C, Q, TC, TQ, gr, gp, tgr, tgp, oc, oq, orr, op, planes}) delete[] p;
  return 0;
}
