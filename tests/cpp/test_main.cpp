// test_main.cpp -- tests of the C++17 drop-in API (include/engine/*.hpp).
//
// Suites named cpu_* need no GPU: preconditions are checked on the host before
// any device call, and the allocator / tensor / half / dtype code has host
// paths. Suites named gpu_* run on the MI355X and fail if no device is visible.
// Modelled on the reference's tests/test_kernels.cu:1664-1844 (launch
// contract), tests/test_allocator.cpp, tests/test_tensor.cpp and
// tests/test_dtype.cpp.
#include <engine/allocator.hpp>
#include <engine/device_buffer.hpp>
#include <engine/dtype.hpp>
#include <engine/engref.hpp>
#include <engine/half.hpp>
#include <engine/hip_device.hpp>
#include <engine/hip_stream.hpp>
#include <engine/kernels.hpp>
#include <engine/pool_allocator.hpp>
#include <engine/tensor.hpp>

#include "mini_test.hpp"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <string>
#include <unistd.h>
#include <vector>

using engine::Device;
using engine::DType;
using engine::Tensor;

namespace {

// ------------------------------------------------------------ launch contract
// Dummy non-null "device" pointers: never dereferenced, because every
// precondition is checked before a launch and zero-size work launches nothing.
float g_dummy_f[16];
engine::half g_dummy_h[16];

TEST(cpu_contract, launchers_reject_negative_dimensions) {
  float* p = g_dummy_f;
  engine::half* ph = g_dummy_h;
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm(p, p, p, -1, 4, 1e-5f), "negative");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, p, p, -1, 4, 4, 1e-5f), "negative");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, p, p, 4, -1, 4, 1e-5f), "negative");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, p, p, 4, 4, -1, 1e-5f), "negative");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, ph, p, 4, 4, -1, 1e-5f), "negative");
  EXPECT_THROWS_MSG(engine::cuda::gemv(p, p, p, -1, 4), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::gemv(p, p, p, 4, -1), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::gemv_fp16(ph, ph, ph, -1, 4), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::gemv_fp16(ph, ph, ph, 4, -1), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::gemv_fp16(ph, p, p, 4, -1), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::matmul_register_tiled(p, p, p, -1, 4, 4), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::matmul_register_tiled(p, p, p, 4, -1, 4), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::matmul_register_tiled(p, p, p, 4, 4, -1), "non-negative");
  // eps < 0 would put a negative number under the square root.
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm(p, p, p, 4, 4, -1.0f), "eps");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, p, p, 4, 4, 4, -1.0f), "eps");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, p, p, 4, 4, 4, std::nanf("")), "eps");
}

TEST(cpu_contract, launchers_reject_null_pointers) {
  float* p = g_dummy_f;
  engine::half* ph = g_dummy_h;
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm(nullptr, p, p, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm(p, p, nullptr, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(nullptr, p, p, p, 2, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, static_cast<const float*>(nullptr), p, 2, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear(p, p, p, nullptr, 2, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::gemv(nullptr, p, p, 4, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::gemv(p, nullptr, p, 4, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::gemv(p, p, nullptr, 4, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::gemv_fp16(nullptr, ph, ph, 4, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::gemv_fp16(ph, static_cast<const engine::half*>(nullptr), ph, 4, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::gemv_fp16(ph, ph, static_cast<engine::half*>(nullptr), 4, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::matmul_register_tiled(nullptr, p, p, 2, 2, 2), "null");
  EXPECT_THROWS_MSG(engine::cuda::matmul_register_tiled(p, nullptr, p, 2, 2, 2), "null");
  EXPECT_THROWS_MSG(engine::cuda::matmul_register_tiled(p, p, nullptr, 2, 2, 2), "null");
  // A null RMSNorm gain is a valid configuration, not a mistake.
  EXPECT_NO_THROW(engine::cuda::rmsnorm(p, nullptr, p, 0, 0, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::rmsnorm_linear(p, nullptr, p, p, 0, 0, 0, 1e-5f));
}

TEST(cpu_contract, empty_work_is_a_no_op_not_an_error) {
  float* p = g_dummy_f;
  engine::half* ph = g_dummy_h;
  EXPECT_NO_THROW(engine::cuda::rmsnorm(p, p, p, 0, 8, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::rmsnorm(p, p, p, 8, 0, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::rmsnorm_linear(p, p, p, p, 0, 8, 8, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::rmsnorm_linear(p, p, p, p, 8, 0, 8, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::rmsnorm_linear(p, p, p, p, 8, 8, 0, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::gemv(p, p, p, 0, 8));
  EXPECT_NO_THROW(engine::cuda::gemv_fp16(ph, ph, ph, 0, 8));
  EXPECT_NO_THROW(engine::cuda::matmul_register_tiled(p, p, p, 0, 8, 8));
  EXPECT_NO_THROW(engine::cuda::matmul_register_tiled(p, p, p, 8, 0, 8));
  for (float v : g_dummy_f) EXPECT_EQ(v, 0.0f);
}

TEST(cpu_contract, ffn_side_launchers_keep_the_reference_contract) {
  float* p = g_dummy_f;
  engine::half* ph = g_dummy_h;
  // reference tests/test_kernels.cu:1679-1839, the rows for these launchers
  EXPECT_THROWS_MSG(engine::cuda::vector_add(p, p, p, -1), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::vector_add(nullptr, p, p, 4), "null");
  EXPECT_NO_THROW(engine::cuda::vector_add(nullptr, nullptr, nullptr, 0));
  EXPECT_THROWS_MSG(engine::cuda::residual_rmsnorm(p, p, p, p, p, -1, 4, 1e-5f), "negative");
  EXPECT_THROWS_MSG(engine::cuda::residual_rmsnorm(p, p, p, p, p, 4, -1, 1e-5f), "negative");
  EXPECT_THROWS_MSG(engine::cuda::residual_rmsnorm(p, p, p, p, p, 4, 4, -1.0f), "eps");
  EXPECT_THROWS_MSG(engine::cuda::residual_rmsnorm(nullptr, p, p, p, p, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::residual_rmsnorm(p, nullptr, p, p, p, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::residual_rmsnorm(p, p, p, nullptr, p, 2, 2, 1e-5f), "null");
  EXPECT_THROWS_MSG(engine::cuda::residual_rmsnorm(p, p, p, p, nullptr, 2, 2, 1e-5f), "null");
  EXPECT_NO_THROW(engine::cuda::residual_rmsnorm(p, p, nullptr, p, p, 0, 0, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::residual_rmsnorm(p, p, p, p, p, 0, 8, 1e-5f));
  EXPECT_NO_THROW(engine::cuda::residual_rmsnorm(p, p, p, p, p, 8, 0, 1e-5f));
  EXPECT_THROWS_MSG(engine::cuda::swiglu(p, p, p, -1), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::swiglu_fp16(ph, ph, ph, -1), "non-negative");
  EXPECT_THROWS_MSG(engine::cuda::swiglu(nullptr, p, p, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::swiglu(p, nullptr, p, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::swiglu(p, p, nullptr, 4), "null");
  EXPECT_THROWS_MSG(engine::cuda::swiglu_fp16(nullptr, ph, ph, 4), "null");
  EXPECT_NO_THROW(engine::cuda::swiglu(p, p, p, 0));
  EXPECT_NO_THROW(engine::cuda::swiglu_fp16(ph, ph, ph, 0));
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear_swiglu_nk(p, p, ph, ph, p, 1, -1, 4, 1e-5f),
                    "negative");
  EXPECT_NO_THROW(engine::cuda::rmsnorm_linear_swiglu_nk(p, nullptr, p, p, p, 1, 8, 0, 1e-5f));
  EXPECT_THROWS_MSG(engine::cuda::rmsnorm_linear_swiglu(p, p, ph, nullptr, p, 1, 4, 4, 1e-5f),
                    "null");
  EXPECT_NO_THROW(engine::cuda::rmsnorm_linear_swiglu(p, nullptr, p, p, p, 0, 8, 8, 1e-5f));
  for (float v : g_dummy_f) EXPECT_EQ(v, 0.0f);
}

TEST(cpu_contract, error_message_layout) {
  try {
    engine::cuda::gemv(nullptr, g_dummy_f, g_dummy_f, 4, 4);
    ctx.fail(__FILE__, __LINE__, "expected a throw");
  } catch (const engine::EngineError& e) {
    const std::string m = e.what();
    EXPECT_TRUE(m.rfind("[engine] ", 0) == 0);
    EXPECT_TRUE(m.find("\n  check failed: ") != std::string::npos);
    EXPECT_TRUE(m.find("gemv: A is null") != std::string::npos);
  }
}

// ------------------------------------------------------------------- allocator
TEST(cpu_allocator, pool_allocates_aligned_blocks) {
  engine::PoolAllocator pool(Device::CPU, 64 * 1024);
  void* p1 = pool.allocate(100);
  ASSERT_TRUE(p1 != nullptr);
  EXPECT_EQ(reinterpret_cast<std::uintptr_t>(p1) % 256, 0u);
  void* p2 = pool.allocate(5000);
  ASSERT_TRUE(p2 != nullptr);
  EXPECT_EQ(reinterpret_cast<std::uintptr_t>(p2) % 256, 0u);
  pool.deallocate(p1);
  pool.deallocate(p2);
}

TEST(cpu_allocator, pool_recycles_freed_memory_blocks) {
  engine::PoolAllocator pool(Device::CPU, 64 * 1024);
  void* p1 = pool.allocate(1024);
  EXPECT_EQ(pool.stats().num_driver_allocs, 1u);
  pool.deallocate(p1);
  EXPECT_EQ(pool.stats().bytes_in_use, 0u);
  void* p2 = pool.allocate(1024);
  EXPECT_EQ(p1, p2);
  EXPECT_EQ(pool.stats().num_driver_allocs, 1u);
  EXPECT_EQ(pool.stats().num_allocs, 2u);
  pool.deallocate(p2);
}

TEST(cpu_allocator, tracks_exact_bytes_in_use_and_peak) {
  engine::PoolAllocator pool(Device::CPU, 64 * 1024);
  void* a = pool.allocate(1024);
  void* b = pool.allocate(2048);
  EXPECT_EQ(pool.stats().bytes_in_use, 3072u);
  EXPECT_EQ(pool.stats().peak_bytes_in_use, 3072u);
  pool.deallocate(a);
  EXPECT_EQ(pool.stats().bytes_in_use, 2048u);
  void* c = pool.allocate(4096);
  EXPECT_EQ(pool.stats().bytes_in_use, 6144u);
  EXPECT_EQ(pool.stats().peak_bytes_in_use, 6144u);
  pool.deallocate(b);
  pool.deallocate(c);
  EXPECT_EQ(pool.stats().bytes_in_use, 0u);
  EXPECT_EQ(pool.stats().peak_bytes_in_use, 6144u);
}

TEST(cpu_allocator, acceptance_100k_cycles_one_driver_alloc) {
  engine::PoolAllocator pool(Device::CPU, 64 * 1024);
  for (int i = 0; i < 100000; ++i) pool.deallocate(pool.allocate(512));
  const auto s = pool.stats();
  EXPECT_EQ(s.num_allocs, 100000u);
  EXPECT_EQ(s.num_driver_allocs, 1u);
  EXPECT_EQ(s.bytes_in_use, 0u);
}

TEST(cpu_allocator, scoped_pool_buffer_frees_on_exception) {
  engine::PoolAllocator pool(Device::CPU, 64 * 1024);
  try {
    engine::ScopedPoolBuffer scratch(pool, 4096);
    EXPECT_EQ(pool.stats().bytes_in_use, 4096u);
    throw std::runtime_error("simulated failure");
  } catch (const std::runtime_error&) {
  }
  EXPECT_EQ(pool.stats().bytes_in_use, 0u);
}

TEST(cpu_allocator, slabs_double_then_cap_and_reset) {
  engine::PoolAllocator pool(Device::CPU, 256 * 1024);
  void* a = pool.allocate(256 * 1024);   // fills slab 1 (256 KiB)
  void* b = pool.allocate(1024);         // new slab of 512 KiB
  EXPECT_EQ(pool.stats().bytes_reserved, 768u * 1024u);
  void* c = pool.allocate(512 * 1024);   // does not fit the 511 KiB left: 1 MiB slab
  EXPECT_EQ(pool.stats().num_driver_allocs, 3u);
  EXPECT_EQ(pool.stats().bytes_reserved, (768u + 1024u) * 1024u);
  pool.deallocate(a);
  pool.deallocate(b);
  pool.deallocate(c);
  pool.reset();
  EXPECT_EQ(pool.stats().bytes_reserved, 0u);
  EXPECT_EQ(pool.stats().num_allocs, 0u);
}

TEST(cpu_allocator, foreign_pointer_is_rejected) {
  engine::PoolAllocator pool(Device::CPU, 64 * 1024);
  int x = 0;
  EXPECT_THROWS_MSG(pool.deallocate(&x), "not allocated by this pool");
}

TEST(cpu_allocator, passthrough_counts_every_request) {
  auto& a = engine::default_allocator(Device::CPU);
  const auto before = a.stats();
  void* p = a.allocate(1000);
  EXPECT_EQ(reinterpret_cast<std::uintptr_t>(p) % 256, 0u);
  a.deallocate(p);
  EXPECT_EQ(a.stats().num_driver_allocs, before.num_driver_allocs + 1);
  EXPECT_TRUE(a.allocate(0) == nullptr);
}

// ---------------------------------------------------------------------- tensor
TEST(cpu_tensor, contiguous_strides_and_numel) {
  Tensor t({2, 3, 4}, DType::F32, Device::CPU);
  EXPECT_EQ(t.strides()[0], 12);
  EXPECT_EQ(t.strides()[1], 4);
  EXPECT_EQ(t.strides()[2], 1);
  EXPECT_EQ(t.numel(), 24);
  EXPECT_EQ(t.nbytes(), 96u);
  EXPECT_TRUE(t.is_contiguous());
  EXPECT_EQ(Tensor().numel(), 0);
  EXPECT_EQ(Tensor({}, DType::F32, Device::CPU).numel(), 1);
  EXPECT_EQ(Tensor({3, 0, 2}, DType::F32, Device::CPU).numel(), 0);
  EXPECT_EQ(Tensor({5}, DType::I4, Device::CPU).nbytes(), 3u);
  EXPECT_EQ(t.size(-1), 4);
  EXPECT_THROWS_MSG(t.size(3), "out of range");
  EXPECT_THROWS_MSG(Tensor({2, -1}, DType::F32, Device::CPU), "must be >= 0");
}

TEST(cpu_tensor, reshape_infers_and_checks) {
  Tensor t({2, 3, 4}, DType::F32, Device::CPU);
  Tensor r = t.reshape({-1, 4});
  EXPECT_EQ(r.shape()[0], 6);
  EXPECT_TRUE(r.storage() == t.storage());
  EXPECT_THROWS_MSG(t.reshape({5, -1}), "cannot infer");
  EXPECT_THROWS_MSG(t.reshape({-1, -1}), "at most one");
  EXPECT_THROWS_MSG(t.reshape({7, 4}), "cannot reshape");
  EXPECT_THROWS_MSG(t.transpose(0, 2).reshape({24}), "contiguous");
}

TEST(cpu_tensor, permute_transpose_slice_are_views) {
  Tensor t({2, 3, 4}, DType::F32, Device::CPU);
  float* d = t.ptr<float>(Device::CPU);
  for (int i = 0; i < 24; ++i) d[i] = static_cast<float>(i);
  Tensor tt = t.transpose(0, 2);  // [4,3,2]
  EXPECT_EQ(tt.shape()[0], 4);
  EXPECT_EQ(tt.strides()[0], 1);
  EXPECT_EQ(tt.strides()[2], 12);
  EXPECT_TRUE(!tt.is_contiguous());
  Tensor c = tt.contiguous();
  const float* cd = c.ptr<float>(Device::CPU);
  // element (i,j,k) of tt is t(k,j,i) = 12k + 4j + i
  bool ok = true;
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 3; ++j)
      for (int k = 0; k < 2; ++k) ok = ok && cd[i * 6 + j * 2 + k] == static_cast<float>(12 * k + 4 * j + i);
  EXPECT_TRUE(ok);
  Tensor s = t.slice(1, 1, 2);  // [2,2,4]
  EXPECT_EQ(s.storage_offset(), 4);
  EXPECT_EQ(*s.ptr<float>(Device::CPU), 4.0f);
  EXPECT_TRUE(!s.is_contiguous());
  EXPECT_THROWS_MSG(t.slice(1, 2, 2), "axis size");
  EXPECT_THROWS_MSG(t.permute({0, 0, 1}), "more than once");
  EXPECT_THROWS_MSG(t.permute({0, 1}), "perm length");
}

TEST(cpu_tensor, clone_from_blob_ptr_and_to_string) {
  float host[6] = {1, 2, 3, 4, 5, 6};
  Tensor b = Tensor::from_blob(host, {2, 3}, DType::F32, Device::CPU);
  EXPECT_TRUE(!b.storage()->owns());
  EXPECT_EQ(b.ptr<float>(Device::CPU), host);
  Tensor c = b.clone();
  EXPECT_TRUE(c.storage()->owns());
  host[0] = 9;
  EXPECT_EQ(c.ptr<float>(Device::CPU)[0], 1.0f);
  EXPECT_THROWS_MSG(b.ptr<double>(Device::CPU), "does not match");
  EXPECT_THROWS_MSG(b.ptr<float>(Device::HIP), "expected device");
  EXPECT_EQ(b.to_string(), std::string("Tensor(f32 on cpu, shape [2, 3], strides [3, 1], offset 0, contiguous)"));
  EXPECT_EQ(b.transpose(0, 1).slice(0, 1, 2).to_string(),
            std::string("Tensor(f32 on cpu, shape [2, 2], strides [1, 3], offset 1, non-contiguous)"));
  Tensor z = Tensor::zeros({3}, DType::F16, Device::CPU);
  EXPECT_EQ(z.ptr<engine::half>(Device::CPU)[2].u, 0u);
  EXPECT_EQ(Tensor().to_string(), std::string("Tensor(undefined)"));
}

namespace {
void fill_ramp(Tensor& t) {
  float* p = t.ptr<float>(Device::CPU);
  for (std::int64_t i = 0; i < t.numel(); ++i) p[i] = static_cast<float>(i);
}
float at2(const Tensor& t, std::int64_t i, std::int64_t j) {
  const float* base = static_cast<const float*>(t.data());
  return base[i * t.strides()[0] + j * t.strides()[1]];
}
}  // namespace

// Behaviours the reference's tensor tests pin (tests/test_tensor.cpp:287-625).
TEST(cpu_tensor, views_share_storage_and_read_through_strides) {
  Tensor t({2, 6}, DType::F32, Device::CPU);
  fill_ramp(t);
  Tensor r = t.reshape({3, 4});
  EXPECT_TRUE(r.strides() == (std::vector<std::int64_t>{4, 1}));
  EXPECT_EQ(at2(r, 1, 1), 5.0f);
  r.ptr<float>(Device::CPU)[0] = 99.0f;
  EXPECT_EQ(static_cast<const float*>(t.data())[0], 99.0f);
  Tensor small({2, 3}, DType::F32, Device::CPU);
  fill_ramp(small);
  Tensor tr = small.transpose(0, 1);
  EXPECT_TRUE(tr.strides() == (std::vector<std::int64_t>{1, 3}));
  EXPECT_EQ(at2(tr, 0, 1), 3.0f);
  EXPECT_EQ(at2(tr, 2, 1), 5.0f);
  Tensor back = tr.transpose(0, 1);
  EXPECT_TRUE(back.strides() == small.strides() && back.is_contiguous());
  Tensor t3({2, 3, 4}, DType::F32, Device::CPU);
  Tensor a = t3.transpose(-1, -2);
  EXPECT_TRUE(a.shape() == (std::vector<std::int64_t>{2, 4, 3}));
  EXPECT_TRUE(a.strides() == (std::vector<std::int64_t>{12, 1, 4}));
  EXPECT_THROWS_MSG(t3.transpose(0, 3), "out of range");
  Tensor p = t3.permute({2, 0, 1});
  EXPECT_TRUE(p.strides() == (std::vector<std::int64_t>{1, 12, 4}));
  EXPECT_TRUE(!p.is_contiguous());
  EXPECT_TRUE(t3.permute({0, 1, 2}).is_contiguous());
  EXPECT_THROWS_MSG(t3.permute({0, 1, 3}), "not a permutation");
  EXPECT_THROWS_MSG(t3.permute({0, 1, 2, 0}), "perm length");
  EXPECT_THROWS_MSG(t3.permute({0, 1}), "perm length");
}

TEST(cpu_tensor, slices_compose_and_allow_empty) {
  Tensor t({4, 5}, DType::F32, Device::CPU);
  fill_ramp(t);
  Tensor rows = t.slice(0, 1, 2);
  EXPECT_EQ(rows.storage_offset(), 5);
  EXPECT_TRUE(rows.is_contiguous());
  EXPECT_EQ(at2(rows, 1, 4), 14.0f);
  Tensor cols = t.slice(1, 2, 2);
  EXPECT_TRUE(cols.strides() == (std::vector<std::int64_t>{5, 1}));
  EXPECT_TRUE(!cols.is_contiguous());
  EXPECT_EQ(at2(cols, 3, 1), 18.0f);
  EXPECT_THROWS_MSG(t.slice(0, 3, 2), "axis size");
  EXPECT_THROWS_MSG(t.slice(0, -1, 2), ">= 0");
  EXPECT_THROWS_MSG(t.slice(0, 0, -1), ">= 0");
  EXPECT_THROWS_MSG(t.slice(2, 0, 1), "out of range");
  EXPECT_NO_THROW(t.slice(-1, 0, 5));
  Tensor sq({6, 6}, DType::F32, Device::CPU);
  fill_ramp(sq);
  Tensor s2 = sq.slice(0, 2, 3).slice(0, 1, 1);
  EXPECT_EQ(s2.storage_offset(), 18);
  EXPECT_EQ(at2(s2, 0, 0), 18.0f);
  Tensor cache({32, 2048, 128}, DType::F32, Device::CPU);
  Tensor empty = cache.slice(1, 0, 0);
  EXPECT_EQ(empty.numel(), 0);
  EXPECT_TRUE(empty.is_contiguous());
  EXPECT_TRUE(empty.contiguous().storage() == cache.storage());
  EXPECT_NO_THROW(empty.to_string());
}

TEST(cpu_tensor, packing_copies_in_row_major_order) {
  Tensor t({2, 3}, DType::F32, Device::CPU);
  fill_ramp(t);
  Tensor c = t.transpose(0, 1).contiguous();
  const float want[6] = {0, 3, 1, 4, 2, 5};
  bool ok = c.storage() != t.storage() && c.is_contiguous();
  for (int i = 0; i < 6; ++i) ok = ok && c.ptr<float>(Device::CPU)[i] == want[i];
  EXPECT_TRUE(ok);
  Tensor t3({2, 3, 4}, DType::F32, Device::CPU);
  fill_ramp(t3);
  Tensor v = t3.slice(0, 1, 1).permute({0, 2, 1});
  Tensor c3 = v.contiguous();
  ok = c3.is_contiguous() && c3.numel() == 12;
  for (int j = 0; j < 4; ++j)
    for (int k = 0; k < 3; ++k)
      ok = ok && c3.ptr<float>(Device::CPU)[j * 3 + k] == static_cast<float>(12 + k * 4 + j);
  EXPECT_TRUE(ok);
  // A strided innermost axis (every other column) and a rank-0 tensor.
  Tensor w({3, 8}, DType::F16, Device::CPU);
  auto* wh = w.ptr<engine::half>(Device::CPU);
  for (int i = 0; i < 24; ++i) wh[i].u = static_cast<std::uint16_t>(i);
  Tensor odd = w.reshape({12, 2}).slice(1, 1, 1).contiguous();
  ok = odd.numel() == 12;
  for (int i = 0; i < 12; ++i) ok = ok && odd.ptr<engine::half>(Device::CPU)[i].u == 2 * i + 1;
  EXPECT_TRUE(ok);
  Tensor scalar({}, DType::F32, Device::CPU);
  EXPECT_TRUE(scalar.is_contiguous() && scalar.contiguous().storage() == scalar.storage());
  // clone always allocates and is independent in both directions.
  Tensor cl = t.clone();
  EXPECT_TRUE(cl.storage() != t.storage());
  cl.ptr<float>(Device::CPU)[0] = -1.0f;
  EXPECT_EQ(t.ptr<float>(Device::CPU)[0], 0.0f);
  Tensor clt = t.transpose(0, 1).clone();
  EXPECT_EQ(clt.ptr<float>(Device::CPU)[1], 3.0f);
}

TEST(cpu_tensor, lifetime_and_storage) {
  Tensor view;
  {
    Tensor owner({10}, DType::F32, Device::CPU);
    fill_ramp(owner);
    view = owner.slice(0, 5, 5);
    EXPECT_TRUE(owner.storage().use_count() >= 2);
  }
  EXPECT_EQ(view.storage().use_count(), 1);
  EXPECT_EQ(view.ptr<float>(Device::CPU)[4], 9.0f);
  std::vector<float> external(8, 3.5f);
  {
    Tensor b = Tensor::from_blob(external.data(), {8}, DType::F32, Device::CPU);
    EXPECT_TRUE(b.data() == external.data());
  }
  EXPECT_EQ(external[7], 3.5f);
  engine::Storage s(1000, Device::CPU);
  EXPECT_EQ(reinterpret_cast<std::uintptr_t>(s.data()) % 256, 0u);
  EXPECT_TRUE(s.owns());
  engine::Storage z(0, Device::CPU);
  EXPECT_TRUE(z.data() == nullptr);
  EXPECT_THROWS_MSG(Tensor::from_blob(nullptr, {2}, DType::F32, Device::CPU), "null");
  EXPECT_TRUE(Tensor::from_blob(nullptr, {0, 4}, DType::F32, Device::CPU).numel() == 0);
  EXPECT_THROWS_MSG(Tensor().reshape({1}), "undefined");
  Tensor h({4}, DType::F32, Device::CPU);
  EXPECT_TRUE(h.to(Device::CPU).storage() == h.storage());
}

// ------------------------------------------------------------------ half/dtype
TEST(cpu_half, round_to_nearest_even) {
  using engine::float_to_half_bits;
  EXPECT_EQ(float_to_half_bits(1.0f), 0x3c00u);
  EXPECT_EQ(float_to_half_bits(65504.0f), 0x7bffu);
  EXPECT_EQ(float_to_half_bits(65520.0f), 0x7c00u);   // tie rounds to even -> overflow
  EXPECT_EQ(float_to_half_bits(65519.99f), 0x7bffu);
  EXPECT_EQ(float_to_half_bits(1.0f + 1.0f / 2048.0f), 0x3c00u);  // tie to even (down)
  EXPECT_EQ(float_to_half_bits(1.0f + 3.0f / 2048.0f), 0x3c02u);  // tie to even (up)
  EXPECT_EQ(float_to_half_bits(std::ldexp(1.0f, -24)), 0x0001u);  // smallest subnormal
  EXPECT_EQ(float_to_half_bits(std::ldexp(1.0f, -25)), 0x0000u);  // tie to even -> 0
  EXPECT_EQ(float_to_half_bits(std::ldexp(1.5f, -25)), 0x0001u);
  EXPECT_EQ(float_to_half_bits(-0.0f), 0x8000u);
  EXPECT_EQ(engine::half_bits_to_float(0x3555u), 0.333251953125f);
  EXPECT_TRUE(std::isnan(engine::half_bits_to_float(engine::float_to_half_bits(std::nanf("")))));
}

TEST(cpu_dtype, bits_sizes_and_names) {
  EXPECT_EQ(engine::dtype_bits(DType::I4), 4);
  EXPECT_EQ(engine::dtype_storage_bytes(DType::I4, 3), 2u);
  EXPECT_EQ(engine::dtype_size(DType::F16), 2u);
  EXPECT_THROWS_MSG(engine::dtype_size(DType::I4), "sub-byte");
  EXPECT_EQ(engine::quant_block_bytes(DType::I4), 18u);
  EXPECT_EQ(engine::quant_effective_bits(DType::I4), 4.5);
  EXPECT_EQ(std::string(engine::dtype_name(DType::BF16)), std::string("bf16"));
}

// ------------------------------------------------------------------------ GPU
void require_gpu(mt::Context& ctx) {
  if (engine::hip_device_count() == 0) {
    ctx.fail(__FILE__, __LINE__, "no GPU visible");
    throw std::runtime_error("no GPU");
  }
}

TEST(gpu_runtime, device_summary_and_buffer_round_trip) {
  require_gpu(ctx);
  engine::print_hip_device_info();
  EXPECT_TRUE(engine::hip_device_arch().rfind("gfx950", 0) == 0);
  EXPECT_EQ(engine::hip_peak_bandwidth_gbs(), 8000.0);
  std::vector<float> h(1000);
  for (size_t i = 0; i < h.size(); ++i) h[i] = static_cast<float>(i) * 0.5f;
  engine::DeviceBuffer<float> d(h);
  EXPECT_TRUE(d.download() == h);
  d.zero();
  EXPECT_EQ(d.download()[999], 0.0f);
  engine::DeviceBuffer<float> moved(std::move(d));
  EXPECT_TRUE(d.get() == nullptr);
  EXPECT_EQ(moved.size(), 1000u);
  Tensor t({4, 5}, DType::F32, Device::CPU);
  for (int i = 0; i < 20; ++i) t.ptr<float>(Device::CPU)[i] = static_cast<float>(i);
  Tensor g = t.to(Device::CUDA);
  EXPECT_TRUE(g.device() == Device::HIP);
  Tensor back = g.clone().to(Device::CPU);
  EXPECT_EQ(back.ptr<float>(Device::CPU)[19], 19.0f);
  EXPECT_THROWS_MSG(g.transpose(0, 1).contiguous(), "cannot be packed on the device");
  EXPECT_THROWS_MSG(g.transpose(0, 1).to(Device::CPU), "contiguous");
  EXPECT_THROWS_MSG(g.ptr<float>(Device::CPU), "expected device");
  Tensor gz = Tensor::zeros({3, 7}, DType::F16, Device::CUDA);
  Tensor hz = gz.slice(0, 1, 2).to(Device::CPU);
  bool zero = hz.numel() == 14;
  for (int i = 0; i < 14; ++i) zero = zero && hz.ptr<engine::half>(Device::CPU)[i].u == 0;
  EXPECT_TRUE(zero);
  // live clocks: the engine clock is positive (live, or the nominal fallback);
  // the source names what was read
  EXPECT_TRUE(engine::hip_live_sm_clock_mhz() > 0);
  EXPECT_TRUE(engine::hip_live_mem_clock_mhz() >= 0);
  char src[512];
  ENGINE_ABI_CHECK(eng_live_clock_source(src, sizeof(src)));
  EXPECT_TRUE(std::string(src).find("engine clock: ") == 0);
  std::printf("  live clocks: %d / %d MHz (%s)\n", engine::hip_live_sm_clock_mhz(),
              engine::hip_live_mem_clock_mhz(), src);
}

TEST(gpu_runtime, hip_check_kernel_after_a_launch) {
  require_gpu(ctx);
  std::vector<float> A(64 * 32, 0.5f), x(64, 2.0f);
  engine::DeviceBuffer<float> dA(A), dx(x), dy(32);
  engine::cuda::gemv(dA.get(), dx.get(), dy.get(), 32, 64);
  EXPECT_NO_THROW([] { HIP_CHECK_KERNEL(); }());
  HIP_CHECK(hipDeviceSynchronize());
  EXPECT_EQ(dy.download()[31], 64.0f);
  // a HIP error reported through HIP_CHECK carries the runtime's name for it
  EXPECT_THROWS_MSG(HIP_CHECK(hipErrorInvalidValue), "hipErrorInvalidValue");
}

TEST(gpu_allocator, pool_allocates_and_recycles_device_memory) {
  require_gpu(ctx);
  engine::PoolAllocator pool(Device::HIP, 1024 * 1024);
  void* d1 = pool.allocate(4096);
  EXPECT_EQ(reinterpret_cast<std::uintptr_t>(d1) % 256, 0u);
  pool.deallocate(d1);
  ENGINE_ABI_CHECK(eng_device_sync());
  void* d2 = pool.allocate(4096);
  EXPECT_EQ(d1, d2);
  EXPECT_EQ(pool.stats().num_driver_allocs, 1u);
  pool.deallocate(d2);
  ENGINE_ABI_CHECK(eng_device_sync());
}

TEST(gpu_allocator, pool_defers_reuse_until_event_completes) {
  require_gpu(ctx);
  engine::PoolAllocator pool(Device::HIP, 1024 * 1024);
  engine::HipStream s1, s2;
  const std::int64_t n = 2048;
  engine::DeviceBuffer<float> a(n * n), b(n * n), c(n * n);
  a.zero();
  b.zero();
  void* d1 = pool.allocate(4096);
  for (int rep = 0; rep < 8; ++rep) engine::cuda::matmul_register_tiled(a.get(), b.get(), c.get(), n, n, n, s1);
  pool.deallocate(d1, s1);
  engine::HipEvent probe(ENG_EVENT_DISABLE_TIMING);
  probe.record(s1);
  void* d2 = pool.allocate(4096);
  const bool busy = !probe.is_complete();
  if (busy) {
    EXPECT_TRUE(d1 != d2);
    s1.synchronize();
    void* d3 = pool.allocate(4096);
    EXPECT_EQ(d3, d1);
    pool.deallocate(d3, s2);
  } else {
    s1.synchronize();
  }
  pool.deallocate(d2, s2);
  s2.synchronize();
}

TEST(gpu_allocator, stream_wait_orders_cross_stream_dependency) {
  require_gpu(ctx);
  engine::HipStream s1, s2;
  engine::HipEvent ev(ENG_EVENT_DISABLE_TIMING);
  engine::DeviceBuffer<float> buf(1);
  buf.zero();
  ev.record(s1);
  s2.wait(ev);
  s2.synchronize();
  EXPECT_TRUE(ev.is_complete());
  EXPECT_EQ(buf.download()[0], 0.0f);
}

TEST(gpu_kernels, k_zero_gives_zero_outputs_through_cpp_api) {
  require_gpu(ctx);
  const std::vector<float> poison(12, 7.0f);
  engine::DeviceBuffer<float> dA(1), dB(1), dC(poison);
  dA.zero();
  dB.zero();
  engine::cuda::matmul_register_tiled(dA.get(), dB.get(), dC.get(), 4, 3, 0);
  ENGINE_ABI_CHECK(eng_device_sync());
  for (float v : dC.download()) EXPECT_EQ(v, 0.0f);
  engine::DeviceBuffer<float> dy(std::vector<float>(13, 7.0f));
  engine::cuda::gemv(dA.get(), dB.get(), dy.get(), 13, 0);
  ENGINE_ABI_CHECK(eng_device_sync());
  for (float v : dy.download()) EXPECT_EQ(v, 0.0f);
  engine::DeviceBuffer<engine::half> hA(1), hx(1);
  engine::DeviceBuffer<engine::half> hy(std::vector<engine::half>(13, engine::float_to_half(7.0f)));
  hA.zero();
  hx.zero();
  engine::cuda::gemv_fp16(hA.get(), hx.get(), hy.get(), 13, 0);
  ENGINE_ABI_CHECK(eng_device_sync());
  for (engine::half v : hy.download()) EXPECT_EQ(engine::half_to_float(v), 0.0f);
  // rmsnorm_linear with K == 0 writes nothing.
  engine::DeviceBuffer<float> ry(poison);
  engine::cuda::rmsnorm_linear(dA.get(), nullptr, dB.get(), ry.get(), 4, 3, 0, 1e-5f);
  ENGINE_ABI_CHECK(eng_device_sync());
  for (float v : ry.download()) EXPECT_EQ(v, 7.0f);
}

TEST(gpu_kernels, rmsnorm_linear_multi_stream) {
  require_gpu(ctx);
  // Decode (M = 1) and prefill (M = 32) launches interleaved on two
  // non-blocking streams; each result is checked against a double-precision
  // host evaluation (reference tests/test_kernels.cu:1197-1265).
  engine::HipStream sa, sb;
  const std::int64_t K = 512, N = 512;
  const float eps = 1e-5f;
  struct Run {
    std::int64_t m;
    engine::DeviceBuffer<float> in, w, W, out;
    std::vector<double> expected, bound;
  };
  std::vector<Run> runs(6);
  for (int i = 0; i < 6; ++i) {
    Run& r = runs[i];
    r.m = (i % 2 == 0) ? 32 : 1;
    const float seed = static_cast<float>(i + 1) * 1.37f;
    std::vector<float> in(r.m * K), w(K), W(K * N);
    for (size_t j = 0; j < in.size(); ++j) in[j] = std::sin(seed + static_cast<float>(j) * 0.013f);
    for (size_t j = 0; j < w.size(); ++j) w[j] = 0.75f + 0.25f * std::cos(seed + static_cast<float>(j) * 0.031f);
    for (size_t j = 0; j < W.size(); ++j) W[j] = 0.05f * std::cos(seed * 1.7f + static_cast<float>(j) * 0.007f);
    r.expected.assign(r.m * N, 0.0);
    r.bound.assign(r.m * N, 0.0);
    for (std::int64_t row = 0; row < r.m; ++row) {
      double ss = 0;
      for (std::int64_t k = 0; k < K; ++k) ss += double(in[row * K + k]) * in[row * K + k];
      const double s = 1.0 / std::sqrt(ss / K + eps);
      for (std::int64_t n = 0; n < N; ++n) {
        double acc = 0, aabs = 0;
        for (std::int64_t k = 0; k < K; ++k) {
          const double t = double(in[row * K + k]) * s * w[k];
          acc += t * W[k * N + n];
          aabs += std::fabs(t * W[k * N + n]);
        }
        r.expected[row * N + n] = acc;
        // derived bound: (K + 3) u sum|t W| + (K / 2 + 5) u |y|
        r.bound[row * N + n] = (K + 3) * 0x1p-24 * aabs + (K / 2.0 + 5) * 0x1p-24 * std::fabs(acc);
      }
    }
    r.in = engine::DeviceBuffer<float>(in);
    r.w = engine::DeviceBuffer<float>(w);
    r.W = engine::DeviceBuffer<float>(W);
    r.out = engine::DeviceBuffer<float>(static_cast<size_t>(r.m * N));
  }
  for (int i = 0; i < 6; ++i) {
    Run& r = runs[i];
    engine::cuda::rmsnorm_linear(r.in.get(), r.w.get(), r.W.get(), r.out.get(), r.m, N, K, eps,
                                 i % 2 == 0 ? sa.get() : sb.get());
  }
  sa.synchronize();
  sb.synchronize();
  for (int i = 0; i < 6; ++i) {
    const std::vector<float> got = runs[i].out.download();
    int bad = 0;
    for (size_t j = 0; j < got.size(); ++j)
      if (!(std::fabs(got[j] - runs[i].expected[j]) <= runs[i].bound[j])) ++bad;
    EXPECT_EQ(bad, 0);
  }
}

TEST(gpu_kernels, ffn_sub_block_through_cpp_api) {
  // The decode FFN as the engine runs it: fused gate/up + SwiGLU, down
  // projection, residual add; against a double-precision host reference.
  require_gpu(ctx);
  const std::int64_t D = 256, F = 704;
  const float eps = 1e-5f;
  std::vector<float> h(D), w(D), Wg(F * D), Wu(F * D), Wd(D * F);
  std::uint64_t state = 7;
  auto next = [&state]() {
    state = state * 6364136223846793005ULL + 1442695040888963407ULL;
    return static_cast<float>(static_cast<double>(state >> 11) * 0x1p-53 * 2.0 - 1.0);
  };
  for (auto& v : h) v = next();
  for (auto& v : w) v = 1.0f + 0.1f * next();
  for (auto& v : Wg) v = next() / 16.0f;
  for (auto& v : Wu) v = next() / 16.0f;
  for (auto& v : Wd) v = next() / 26.0f;
  engine::DeviceBuffer<float> dh(h), dw(w), dWg(Wg), dWu(Wu), dWd(Wd);
  engine::DeviceBuffer<float> act(F), down(D), out(D), sum(D), norm(D);
  engine::cuda::rmsnorm_linear_swiglu_nk(dh.get(), dw.get(), dWg.get(), dWu.get(), act.get(), 1, F,
                                         D, eps);
  engine::cuda::gemv_nk(dWd.get(), act.get(), down.get(), D, F);
  engine::cuda::vector_add(dh.get(), down.get(), out.get(), D);
  engine::cuda::residual_rmsnorm(dh.get(), down.get(), dw.get(), norm.get(), sum.get(), 1, D, eps);
  ENGINE_ABI_CHECK(eng_device_sync());

  double ss = 0.0;
  for (float v : h) ss += static_cast<double>(v) * v;
  const double s = 1.0 / std::sqrt(ss / D + eps);
  std::vector<double> a(F);
  for (std::int64_t n = 0; n < F; ++n) {
    double g = 0.0, u = 0.0;
    for (std::int64_t k = 0; k < D; ++k) {
      const double xs = h[k] * s * w[k];
      g += xs * Wg[n * D + k];
      u += xs * Wu[n * D + k];
    }
    a[n] = g / (1.0 + std::exp(-g)) * u;
  }
  const std::vector<float> got_out = out.download();
  const std::vector<float> got_sum = sum.download();
  const std::vector<float> got_down = down.download();
  int bad = 0;
  for (std::int64_t d = 0; d < D; ++d) {
    double dn = 0.0, dabs = 0.0;
    for (std::int64_t f = 0; f < F; ++f) {
      dn += a[f] * Wd[d * F + f];
      dabs += std::fabs(a[f] * Wd[d * F + f]);
    }
    // generous derived bound: (D + F) u over the absolute sums of both stages
    const double bound = (D + F + 8) * 0x1p-24 * (dabs + std::fabs(h[d]) + 1.0);
    if (!(std::fabs(got_out[d] - (h[d] + dn)) <= bound)) ++bad;
    // residual_rmsnorm's sum_out is the same fp32 addition as vector_add
    if (got_sum[d] != h[d] + got_down[d]) ++bad;
  }
  EXPECT_EQ(bad, 0);
  EXPECT_TRUE(got_out == got_sum);
}

// --------------------------------------------------------------------- engref
// Writes an ENGREF01 file (the reference's container, tools/gen_reference.py:
// 64-83) with explicit dtype codes.
struct EngrefWriter {
  std::vector<unsigned char> body;
  int count = 0;
  template <typename T>
  void pod(T v) {
    const auto* p = reinterpret_cast<const unsigned char*>(&v);
    body.insert(body.end(), p, p + sizeof(T));
  }
  void add(const std::string& name, std::int32_t code, std::vector<std::int64_t> dims,
           const void* data, std::int64_t nbytes) {
    pod<std::int32_t>(static_cast<std::int32_t>(name.size()));
    body.insert(body.end(), name.begin(), name.end());
    pod<std::int32_t>(code);
    pod<std::int32_t>(static_cast<std::int32_t>(dims.size()));
    for (auto d : dims) pod<std::int64_t>(d);
    pod<std::int64_t>(nbytes);
    const auto* p = static_cast<const unsigned char*>(data);
    body.insert(body.end(), p, p + nbytes);
    ++count;
  }
  std::string save(const std::string& stem) const {
    const std::string path = "/tmp/engref_cpp_" + std::to_string(::getpid()) + "_" + stem + ".bin";
    std::FILE* f = std::fopen(path.c_str(), "wb");
    std::fwrite("ENGREF01", 1, 8, f);
    std::fwrite(&count, 4, 1, f);
    std::fwrite(body.data(), 1, body.size(), f);
    std::fclose(f);
    return path;
  }
};

TEST(cpu_engref, load_names_dims_and_values) {
  EngrefWriter w;
  const float xs[3] = {1.5f, -2.0f, 3.25f};
  const std::uint16_t hs[4] = {0x3c00, 0xc000, 0x3555, 0x7bff};  // 1, -2, 0.333251953125, 65504
  const double ds[2] = {0.1, -7.0};
  w.add("x", ENG_ENGREF_F32, {3}, xs, sizeof(xs));
  w.add("h", ENG_ENGREF_F16, {2, 2}, hs, sizeof(hs));
  w.add("d", ENG_ENGREF_F64, {2}, ds, sizeof(ds));
  const std::string path = w.save("values");
  engine::EngrefFile f = engine::EngrefFile::load(path);
  EXPECT_EQ(f.size(), 3u);
  EXPECT_TRUE(f.names() == (std::vector<std::string>{"d", "h", "x"}));
  EXPECT_TRUE(f.has("h") && !f.has("y"));
  EXPECT_EQ(f.at("h").dim(1), 2);
  EXPECT_EQ(f.at("h").nbytes, 8);
  EXPECT_THROWS_MSG(f.at("h").dim(2), "out of range");
  EXPECT_TRUE(f.at("x").floats() == (std::vector<float>{1.5f, -2.0f, 3.25f}));
  EXPECT_TRUE(f.at("h").floats() == (std::vector<float>{1.0f, -2.0f, 0.333251953125f, 65504.0f}));
  EXPECT_EQ(f.at("d").floats()[0], 0.1f);
  EXPECT_TRUE(f.at("h").dtype() == DType::F16);
  EXPECT_THROWS_MSG(f.at("d").dtype(), "float64");
  EXPECT_THROWS_MSG(f.at("nope"), "not found. Available: d h x");
  EXPECT_EQ(f.at("x").slab_offset, 0);
  EXPECT_EQ(f.at("h").slab_offset, 256);
  EXPECT_EQ(f.at("d").slab_offset, 512);
  EXPECT_EQ(f.slab_bytes(), 768);
  std::remove(path.c_str());
}

TEST(cpu_engref, errors_follow_the_reference_reader) {
  engine::EngrefFile f;
  std::string err;
  EXPECT_TRUE(!engine::EngrefFile::try_load("/nonexistent/dir/file.bin", f, err));
  EXPECT_TRUE(err.find("cannot open") != std::string::npos);
  EngrefWriter w;
  const float v[2] = {1, 2};
  w.add("t", ENG_ENGREF_F32, {3}, v, sizeof(v));  // 8 bytes for a shape of 3 floats
  const std::string path = w.save("mismatch");
  EXPECT_THROWS_MSG(engine::EngrefFile::load(path), "header says 8 bytes but its shape implies 12");
  std::remove(path.c_str());
  EngrefWriter d;
  d.add("t", ENG_ENGREF_F32, {2}, v, sizeof(v));
  d.add("t", ENG_ENGREF_F32, {2}, v, sizeof(v));
  const std::string dup = d.save("dup");
  EXPECT_THROWS_MSG(engine::EngrefFile::load(dup), "duplicate tensor name 't'");
  std::remove(dup.c_str());
}

TEST(gpu_engref, weight_slab_views_feed_the_reference_api) {
  require_gpu(ctx);
  const std::int64_t K = 640, N = 384;
  std::mt19937 rng(11);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  std::vector<engine::half> A(static_cast<std::size_t>(K * N)), x(static_cast<std::size_t>(K));
  for (auto& a : A) a = engine::float_to_half(0.05f * nd(rng));
  for (auto& v : x) v = engine::float_to_half(nd(rng));
  EngrefWriter w;
  w.add("x", ENG_ENGREF_F16, {K}, x.data(), K * 2);
  w.add("A", ENG_ENGREF_F16, {K, N}, A.data(), K * N * 2);
  const std::string path = w.save("slab");
  engine::EngrefFile f = engine::EngrefFile::load(path);
  engine::WeightSlab slab = engine::WeightSlab::upload(f);
  EXPECT_EQ(static_cast<std::int64_t>(slab.bytes()), f.slab_bytes());
  Tensor tA = slab.tensor("A");
  Tensor tx = slab.tensor("x");
  EXPECT_TRUE(tA.device() == Device::HIP && tA.dtype() == DType::F16);
  EXPECT_TRUE(tA.shape() == (std::vector<std::int64_t>{K, N}));
  EXPECT_TRUE(tA.storage() == tx.storage());  // both alias the one slab
  EXPECT_EQ(tA.data(), slab.data("A"));
  // the slab's bytes are the file's
  Tensor back = tA.to(Device::CPU);
  EXPECT_EQ(std::memcmp(back.data(), A.data(), A.size() * 2), 0);
  engine::DeviceBuffer<engine::half> out(static_cast<std::size_t>(N));
  engine::cuda::gemv_fp16(tA.ptr<engine::half>(Device::HIP), tx.ptr<engine::half>(Device::HIP),
                          out.get(), N, K);
  // the same weights converted to output-major [N x K] on the device
  engine::DeviceBuffer<engine::half> W(static_cast<std::size_t>(N * K));
  engine::cuda::transpose(tA.ptr<engine::half>(Device::HIP), W.get(), K, N);
  const std::vector<engine::half> wt = W.download();
  int moved_wrong = 0;
  for (std::int64_t k = 0; k < K; ++k)
    for (std::int64_t n = 0; n < N; ++n) moved_wrong += wt[n * K + k].u != A[k * N + n].u;
  EXPECT_EQ(moved_wrong, 0);
  HIP_CHECK(hipDeviceSynchronize());
  const std::vector<engine::half> got = out.download();
  int bad = 0;
  for (std::int64_t n = 0; n < N; ++n) {
    double ref = 0.0, mag = 0.0;
    for (std::int64_t k = 0; k < K; ++k) {
      const double p = double(engine::half_to_float(x[k])) * engine::half_to_float(A[k * N + n]);
      ref += p;
      mag += std::fabs(p);
    }
    // fp32 accumulation (K u sum|p|) plus the half rounding of the output
    const double bound = K * 0x1p-24 * mag + 0x1p-11 * std::fabs(ref);
    if (!(std::fabs(engine::half_to_float(got[n]) - ref) <= bound)) ++bad;
  }
  EXPECT_EQ(bad, 0);
  std::remove(path.c_str());
}

}  // namespace

int main(int argc, char** argv) { return mt::run_all(argc, argv); }
