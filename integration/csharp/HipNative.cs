// LibraryImport declarations of libsimdyolo_hip (include/simdyolo_hip.h).
//
// NOT BUILT IN THIS REPOSITORY: the image that builds the HIP library has no
// .NET SDK.  This file, HipBackend.cs and IFastPathBackend.cs are source for
// the reference's src/SimdYolo/ (which already compiles with
// AllowUnsafeBlocks for its Vulkan backend); the library is found as
// "simdyolo_hip" on the native loader path (libsimdyolo_hip.so).
//
// Struct layouts mirror the C header field for field (sequential, natural
// alignment); status codes map to the exception types the Vulkan backend
// raises (VulkanBackend.cs:323, VulkanExecution.cs:229).
using System.Runtime.InteropServices;

namespace SimdYolo;

[StructLayout(LayoutKind.Sequential)]
internal struct SyTensor { public nint Data; public int N, C, H, W, Ldc, Layout; }

[StructLayout(LayoutKind.Sequential)]
internal struct SyModelConfig { public int Arch; public float Depth, Width; public int MaxChannels, Nc, RegMax; public float BnEps; public int Nm, Npr; }

[StructLayout(LayoutKind.Sequential)]
internal struct SyLetterbox { public int SourceWidth, SourceHeight, TargetWidth, TargetHeight; public float ScaleX, ScaleY; public int PadX, PadY; }

[StructLayout(LayoutKind.Sequential)]
internal struct SyDetection { public int ClassId; public float Confidence, X, Y, Width, Height; public int Anchor; }

[StructLayout(LayoutKind.Sequential)]
internal struct SyDecodeOptions { public float Confidence, Iou; public int MaxDetections, MaxCandidates, ClassCount, Agnostic, Layout; }

[StructLayout(LayoutKind.Sequential)]
internal struct SyMaskInfo { public int Left, Top, Width, Height; public long Offset; }

internal static unsafe partial class HipNative
{
    private const string Lib = "simdyolo_hip";

    internal const int LayoutNhwc = 0, LayoutNchw = 1;
    internal const int ArchYolov8 = 0, ArchYolo11 = 1, ArchYolo26 = 2;

    // ------------------------------------------------------------ lifecycle, frames, memory
    [LibraryImport(Lib, EntryPoint = "sy_create")] internal static partial int Create(int device, out nint ctx);
    [LibraryImport(Lib, EntryPoint = "sy_destroy")] internal static partial void Destroy(nint ctx);
    [LibraryImport(Lib, EntryPoint = "sy_name")] internal static partial nint Name(nint ctx);
    [LibraryImport(Lib, EntryPoint = "sy_last_error")] internal static partial nint LastError();
    [LibraryImport(Lib, EntryPoint = "sy_device_count")] internal static partial int DeviceCount(out int count);
    [LibraryImport(Lib, EntryPoint = "sy_frame_begin")] internal static partial int FrameBegin(nint ctx, out long frameId);
    [LibraryImport(Lib, EntryPoint = "sy_frame_end")] internal static partial int FrameEnd(nint ctx);
    [LibraryImport(Lib, EntryPoint = "sy_flush")] internal static partial int Flush(nint ctx);
    [LibraryImport(Lib, EntryPoint = "sy_frame_alloc")] internal static partial int FrameAlloc(nint ctx, int n, int c, int h, int w, out SyTensor view);
    [LibraryImport(Lib, EntryPoint = "sy_upload_nchw")] internal static partial int UploadNchw(nint ctx, float* host, in SyTensor dst);
    [LibraryImport(Lib, EntryPoint = "sy_download_nchw")] internal static partial int DownloadNchw(nint ctx, in SyTensor src, float* host);
    [LibraryImport(Lib, EntryPoint = "sy_malloc")] internal static partial int Malloc(nint ctx, nuint bytes, out nint ptr);
    [LibraryImport(Lib, EntryPoint = "sy_free")] internal static partial int Free(nint ctx, nint ptr);
    // kind: 0 host->device, 1 device->host, 2 device->device; host copies return once the host buffer is done.
    [LibraryImport(Lib, EntryPoint = "sy_memcpy")] internal static partial int Memcpy(nint ctx, nint dst, nint src, nuint bytes, int kind);

    // ------------------------------------------------------------ convolution
    [LibraryImport(Lib, EntryPoint = "sy_conv_create")]
    internal static partial int ConvCreate(nint ctx, float* w, float* bias, int oc, int ic, int kh, int kw,
        int sh, int sw, int pt, int pl, int pb, int pr, int dh, int dw, int groups, int silu, out ulong conv);
    [LibraryImport(Lib, EntryPoint = "sy_conv_transpose2x2_create")]
    internal static partial int ConvTranspose2x2Create(nint ctx, float* wIohw, float* bias, int ic, int oc, out ulong conv);
    [LibraryImport(Lib, EntryPoint = "sy_conv_run")] internal static partial int ConvRun(nint ctx, ulong conv, in SyTensor x, in SyTensor y, SyTensor* residual);
    [LibraryImport(Lib, EntryPoint = "sy_conv_run_upsampled")] internal static partial int ConvRunUpsampled(nint ctx, ulong conv, in SyTensor xu, in SyTensor x, in SyTensor y, SyTensor* residual);
    [LibraryImport(Lib, EntryPoint = "sy_conv_out_size")] internal static partial int ConvOutSize(nint ctx, ulong conv, int h, int w, out int oh, out int ow);
    [LibraryImport(Lib, EntryPoint = "sy_conv_set_algo")] internal static partial int ConvSetAlgo(nint ctx, ulong conv, int algo);
    // Autotuner decisions as a text table (the persisted counterpart of VulkanPipelineCache.cs).
    [LibraryImport(Lib, EntryPoint = "sy_tune_save", StringMarshalling = StringMarshalling.Utf8)] internal static partial int TuneSave(nint ctx, string path);
    [LibraryImport(Lib, EntryPoint = "sy_tune_load", StringMarshalling = StringMarshalling.Utf8)] internal static partial int TuneLoad(nint ctx, string path);

    // ------------------------------------------------------------ fused YOLO ops
    [LibraryImport(Lib, EntryPoint = "sy_add")] internal static partial int Add(nint ctx, in SyTensor a, in SyTensor b, in SyTensor y);
    [LibraryImport(Lib, EntryPoint = "sy_resize_nearest")] internal static partial int ResizeNearest(nint ctx, in SyTensor x, in SyTensor y);
    [LibraryImport(Lib, EntryPoint = "sy_sppf_pool")] internal static partial int SppfPool(nint ctx, in SyTensor x, in SyTensor y5, in SyTensor y9, in SyTensor y13);
    [LibraryImport(Lib, EntryPoint = "sy_copy")] internal static partial int Copy(nint ctx, in SyTensor x, in SyTensor y);
    [LibraryImport(Lib, EntryPoint = "sy_detect_decode")]
    internal static partial int DetectDecode(nint ctx, SyTensor* levels, float* strides, int nLevels, int bins, int nc, int xyxy, nint output, int total);
    [LibraryImport(Lib, EntryPoint = "sy_e2e_topk")]
    internal static partial int EndToEndTopK(nint ctx, nint head, int batch, int channels, int anchors, int nc, int maximum, int onnxRules, nint output);
    // Same results without device allocation (a fixed 32 MiB block per GPU): for frames under graph capture.
    [LibraryImport(Lib, EntryPoint = "sy_e2e_topk_noalloc")]
    internal static partial int EndToEndTopKNoAlloc(nint ctx, nint head, int batch, int channels, int anchors, int nc, int maximum, int onnxRules, nint output);
    [LibraryImport(Lib, EntryPoint = "sy_attention")]
    internal static partial int Attention(nint ctx, in SyTensor qkv, int heads, int keyDim, int headDim, float scale, in SyTensor o, in SyTensor v);

    // ------------------------------------------------------------ generic device ops
    // IDeviceBackend.Compute: one tensor.comp operation; inputs[3] / lengths[3] are the A, B, D bindings.
    [LibraryImport(Lib, EntryPoint = "sy_compute")]
    internal static partial int Compute(nint ctx, int op, nint* inputs, nuint* lengths, uint* parameters, long workItems, nint output, nuint outputLength);
    // IDeviceBackend.DeviceMatMul: batched row-major products with per-axis matrix strides (0 = broadcast).
    [LibraryImport(Lib, EntryPoint = "sy_matmul")]
    internal static partial int MatMul(nint ctx, nint a, nint b, nint c, int m, int n, int k, int batchRank,
        int* batchShape, long* aBatchStrides, long* bBatchStrides, nuint aLength, nuint bLength, nuint cLength);

    // ------------------------------------------------------------ graphs
    [LibraryImport(Lib, EntryPoint = "sy_graph_begin")] internal static partial int GraphBegin(nint ctx);
    [LibraryImport(Lib, EntryPoint = "sy_graph_end")] internal static partial int GraphEnd(nint ctx, out ulong graph);
    [LibraryImport(Lib, EntryPoint = "sy_graph_launch")] internal static partial int GraphLaunch(nint ctx, ulong graph);
    [LibraryImport(Lib, EntryPoint = "sy_graph_destroy")] internal static partial int GraphDestroy(nint ctx, ulong graph);

    // ------------------------------------------------------------ whole model
    [LibraryImport(Lib, EntryPoint = "sy_model_layout")] internal static partial int ModelLayout(in SyModelConfig cfg, int* output, int maxEntries, out int count);
    [LibraryImport(Lib, EntryPoint = "sy_model_create")]
    internal static partial int ModelCreate(nint ctx, in SyModelConfig cfg, float* parameters, nuint count, out nint model);
    [LibraryImport(Lib, EntryPoint = "sy_model_destroy")] internal static partial void ModelDestroy(nint model);
    // Dims 1 and 2 of the model output.  NMS heads: (channels, anchors) of [batch, nc + 4 (+ nm), anchors].
    // End-to-end models (ArchYolo26): (rows, fields) of the selected [batch, k, 6 (+ nm)], k = min(300, anchors).
    [LibraryImport(Lib, EntryPoint = "sy_model_output_shape")] internal static partial int ModelOutputShape(nint model, int batch, int h, int w, out int channels, out int anchors);
    // The joined head [batch, nc + 4 (+ nm), anchors] on the device; for end-to-end models the head before selection.
    [LibraryImport(Lib, EntryPoint = "sy_model_head")]
    internal static partial int ModelHead(nint model, int batch, int h, int w, out nint head, out int channels, out int anchors);
    [LibraryImport(Lib, EntryPoint = "sy_model_predict_raw")]
    internal static partial int ModelPredictRaw(nint model, float* input, int batch, int h, int w, float* output);
    [LibraryImport(Lib, EntryPoint = "sy_model_predict_seg")]
    internal static partial int ModelPredictSeg(nint model, float* input, int batch, int h, int w, float* output, float* protos);
    [LibraryImport(Lib, EntryPoint = "sy_model_buffers")] internal static partial int ModelBuffers(nint model, int batch, int h, int w, out nint input, out nint output);
    [LibraryImport(Lib, EntryPoint = "sy_model_run")] internal static partial int ModelRun(nint model, int batch, int h, int w);
    [LibraryImport(Lib, EntryPoint = "sy_model_proto")]
    internal static partial int ModelProto(nint model, int batch, int h, int w, out nint protos, out int nm, out int ph, out int pw);
    [LibraryImport(Lib, EntryPoint = "sy_model_set_branch_level")] internal static partial int ModelSetBranchLevel(nint model, int level);
    // Activation arena of one input shape (shared by liveness), what it would be unshared, and its scratch.
    [LibraryImport(Lib, EntryPoint = "sy_model_plan_memory")]
    internal static partial int ModelPlanMemory(nint model, int batch, int h, int w, out nuint arenaBytes, out nuint unsharedBytes, out nuint scratchBytes);

    // ------------------------------------------------------------ pre/post-processing
    [LibraryImport(Lib, EntryPoint = "sy_letterbox_device")]
    internal static partial int LetterboxDevice(nint ctx, nint pixels, int width, int height, int tw, int th, int bgr, int rowStride, nint output, out SyLetterbox t);
    [LibraryImport(Lib, EntryPoint = "sy_decode_detections_device")]
    internal static partial int DecodeDetectionsDevice(nint ctx, nint head, int batch, int channels, int anchors,
        in SyDecodeOptions options, SyLetterbox* transforms, SyDetection* output, int maxOut, int* counts);
    [LibraryImport(Lib, EntryPoint = "sy_mask_decode")]
    internal static partial int MaskDecode(nint ctx, in SyTensor protos, nint coeffs, int ldCoeff, int k,
        SyDetection* boxes, in SyLetterbox t, nint masks, nuint capacity, SyMaskInfo* info);

    // Status -> the exception types the reference raises.
    internal static void Check(int status)
    {
        if (status == 0) return;
        string message = Marshal.PtrToStringUTF8(LastError()) ?? "HIP backend error";
        throw status switch
        {
            1 => new ArgumentException(message),
            2 => new NotSupportedException(message),
            _ => new InvalidOperationException($"HIP {message} (status {status})"),
        };
    }
}
