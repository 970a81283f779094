// Per-atom model rows through LAMMPS' comm buffers on the device (the pair style's
// pack/unpack_{forward,reverse}_comm_kokkos, cpp/pair_jax_kokkos.cpp:523-571, with the row
// functors of cpp:247-318).
//
// A model row is `width` scalars at the contract precision; a buffer row is `slots` doubles,
// slots = ceil(width * scalar bytes / 8), the size LAMMPS reserves per atom (comm_forward /
// comm_reverse, cpp:643-647). The copies move 4-byte words, one thread per word, so a wide
// exchange is one coalesced pass and the bytes arrive unchanged whatever the scalar type; an odd
// word count leaves a pad word, written as zero. The reverse unpack adds scalars (the adjoint of
// the forward copy); LAMMPS' send list of one swap names each row once, so the adds of one launch
// never meet.
//
// Row indices are checked against the row capacity (the contract's max_atoms): an index outside
// it is skipped, never dereferenced.

#include "lk_device.h"
#include "lk_internal.h"

namespace lk {

namespace {

constexpr int kCommBlock = 256;

// buffer row i, word w (a buffer row is 2 * slots words)
__device__ __forceinline__ long buf_word(int i, int w, int slots)
{
  return static_cast<long>(i) * 2 * slots + w;
}

// PackCommWordsByList (cpp:247-264): buf row i <- rows[list[i]].
__global__ __launch_bounds__(kCommBlock) void k_comm_pack_list(const uint32_t *__restrict__ rows,
                                                                const int *__restrict__ list,
                                                                int n, int words, int slots,
                                                                int capacity,
                                                                uint32_t *__restrict__ buf)
{
  const long flat = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (flat >= static_cast<long>(n) * words) return;
  const int i = static_cast<int>(flat / words), w = static_cast<int>(flat % words);
  const int j = list[i];
  if (j >= 0 && j < capacity) buf[buf_word(i, w, slots)] = rows[static_cast<long>(j) * words + w];
  if ((words & 1) && w + 1 == words) buf[buf_word(i, words, slots)] = 0u;
}

// PackCommWordsAt (cpp:283-299): buf row i <- rows[first + i].
__global__ __launch_bounds__(kCommBlock) void k_comm_pack_at(const uint32_t *__restrict__ rows,
                                                              int first, int n, int words,
                                                              int slots,
                                                              uint32_t *__restrict__ buf)
{
  const long flat = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (flat >= static_cast<long>(n) * words) return;
  const int i = static_cast<int>(flat / words), w = static_cast<int>(flat % words);
  buf[buf_word(i, w, slots)] = rows[static_cast<long>(first + i) * words + w];
  if ((words & 1) && w + 1 == words) buf[buf_word(i, words, slots)] = 0u;
}

// UnpackCommWordsAt (cpp:266-281): rows[first + i] <- buf row i.
__global__ __launch_bounds__(kCommBlock) void k_comm_unpack_at(uint32_t *__restrict__ rows,
                                                                int first, int n, int words,
                                                                int slots,
                                                                const uint32_t *__restrict__ buf)
{
  const long flat = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (flat >= static_cast<long>(n) * words) return;
  const int i = static_cast<int>(flat / words), w = static_cast<int>(flat % words);
  rows[static_cast<long>(first + i) * words + w] = buf[buf_word(i, w, slots)];
}

// AddCommRowsByList (cpp:301-317): rows[list[i]] += buf row i, scalar by scalar.
template <typename S>
__global__ __launch_bounds__(kCommBlock) void k_comm_add_list(S *__restrict__ rows,
                                                               const int *__restrict__ list, int n,
                                                               int width, int slots, int capacity,
                                                               const double *__restrict__ buf)
{
  const long flat = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (flat >= static_cast<long>(n) * width) return;
  const int i = static_cast<int>(flat / width), w = static_cast<int>(flat % width);
  const int j = list[i];
  if (j < 0 || j >= capacity) return;
  const S *row = reinterpret_cast<const S *>(buf + static_cast<long>(i) * slots);
  rows[static_cast<long>(j) * width + w] += row[w];
}

dim3 comm_grid(int n, int per_row)
{
  const long threads = static_cast<long>(n) * per_row;
  return dim3(static_cast<unsigned>((threads + kCommBlock - 1) / kCommBlock));
}

}  // namespace

int comm_slots(const Handle &h, int width)
{
  return static_cast<int>((static_cast<long>(width) * h.scalar_bytes() + 7) / 8);
}

hipError_t launch_comm_pack_forward(Handle &h, hipStream_t s, const void *rows, int width,
                                    const int *list, int n, double *buf)
{
  if (n <= 0) return hipSuccess;
  const int words = width * static_cast<int>(h.scalar_bytes() / 4);
  StageTimer timer(h, s, "comm_pack_forward");
  hipLaunchKernelGGL(k_comm_pack_list, comm_grid(n, words), dim3(kCommBlock), 0, s,
                     static_cast<const uint32_t *>(rows), list, n, words, comm_slots(h, width),
                     h.contract.max_atoms, reinterpret_cast<uint32_t *>(buf));
  return hipGetLastError();
}

hipError_t launch_comm_unpack_forward(Handle &h, hipStream_t s, void *rows, int width, int first,
                                      int n, const double *buf)
{
  if (n <= 0) return hipSuccess;
  const int words = width * static_cast<int>(h.scalar_bytes() / 4);
  StageTimer timer(h, s, "comm_unpack_forward");
  hipLaunchKernelGGL(k_comm_unpack_at, comm_grid(n, words), dim3(kCommBlock), 0, s,
                     static_cast<uint32_t *>(rows), first, n, words, comm_slots(h, width),
                     reinterpret_cast<const uint32_t *>(buf));
  return hipGetLastError();
}

hipError_t launch_comm_pack_reverse(Handle &h, hipStream_t s, const void *rows, int width,
                                    int first, int n, double *buf)
{
  if (n <= 0) return hipSuccess;
  const int words = width * static_cast<int>(h.scalar_bytes() / 4);
  StageTimer timer(h, s, "comm_pack_reverse");
  hipLaunchKernelGGL(k_comm_pack_at, comm_grid(n, words), dim3(kCommBlock), 0, s,
                     static_cast<const uint32_t *>(rows), first, n, words, comm_slots(h, width),
                     reinterpret_cast<uint32_t *>(buf));
  return hipGetLastError();
}

hipError_t launch_comm_unpack_reverse(Handle &h, hipStream_t s, void *rows, int width,
                                      const int *list, int n, const double *buf)
{
  if (n <= 0) return hipSuccess;
  const int slots = comm_slots(h, width);
  StageTimer timer(h, s, "comm_unpack_reverse");
  if (h.contract.precision == LK_FLOAT64)
    hipLaunchKernelGGL(k_comm_add_list<double>, comm_grid(n, width), dim3(kCommBlock), 0, s,
                       static_cast<double *>(rows), list, n, width, slots, h.contract.max_atoms,
                       buf);
  else
    hipLaunchKernelGGL(k_comm_add_list<float>, comm_grid(n, width), dim3(kCommBlock), 0, s,
                       static_cast<float *>(rows), list, n, width, slots, h.contract.max_atoms,
                       buf);
  return hipGetLastError();
}

}  // namespace lk
