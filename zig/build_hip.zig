//! build_hip.zig -- build.zig fragment that links the MI355X attention library into the engine.
//!
//! The reference's build.zig compiles CUDA_SRC with nvcc in `cudalize` (build.zig:72-107) when -Dcuda=true.  With
//! -Dhip=true the engine instead:
//!   1. builds libllmgen_attn.so once with hipcc for gfx950 (`python3 -m llmgen_amd.build`, which compiles every
//!      llmgen_amd/csrc/*.hip and *.cpp with packed-FP32 instructions disabled and links one shared library);
//!   2. links it and the HIP runtime into the module;
//!   3. exposes `have_hip` to the sources, so that src/backend/cuda/cuda.zig:14-15 imports PagedAttentionImpl /
//!      FlashAttentionImpl from attention_hip.zig and the context externs from hip_context.zig in place of
//!      attention_v1.zig / cuda_context.zig.  The other CUDA kernels (linear, norm, rope ...) are not part of
//!      this library; an engine built with -Dhip=true runs them from its own HIP build or on the CPU backend.
//!
//! Use from build.zig (next to the existing cuda option, build.zig:20-40):
//!
//!     const hip_build = @import("build_hip.zig");
//!     const with_hip = b.option(bool, "hip", "link the MI355X attention library (gfx950)") orelse false;
//!     opts.addOption(bool, "have_hip", with_hip);
//!     if (with_hip) hip_build.linkHipAttention(b, exe.root_module, .{});
//!
//! Not compiled in this repository (no Zig toolchain).
const std = @import("std");

pub const HipConfig = struct {
    /// repository of this library, relative to the engine's build root
    lib_repo: []const u8 = "third_party/llmgen_amd",
    /// ROCm installation (hipcc, libamdhip64)
    rocm: []const u8 = "/opt/rocm",
    python: []const u8 = "python3",
};

pub fn linkHipAttention(b: *std.Build, mod: *std.Build.Module, cfg: HipConfig) void {
    // hipcc --offload-arch=gfx950 over llmgen_amd/csrc -> llmgen_amd/libllmgen_attn.so
    const build_lib = b.addSystemCommand(&.{ cfg.python, "-m", "llmgen_amd.build" });
    build_lib.setCwd(b.path(cfg.lib_repo));
    build_lib.setEnvironmentVariable("HIPCC", b.fmt("{s}/bin/hipcc", .{cfg.rocm}));
    b.getInstallStep().dependOn(&build_lib.step);

    const lib_dir = b.path(b.fmt("{s}/llmgen_amd", .{cfg.lib_repo}));
    mod.addLibraryPath(lib_dir);
    mod.addRPath(lib_dir);
    mod.linkSystemLibrary("llmgen_attn", .{});
    mod.addLibraryPath(.{ .cwd_relative = b.fmt("{s}/lib", .{cfg.rocm}) });
    mod.linkSystemLibrary("amdhip64", .{});
    for ([_][]const u8{ "stdc++", "m", "pthread", "dl", "rt" }) |lib| mod.linkSystemLibrary(lib, .{});
    mod.link_libc = true;
}
