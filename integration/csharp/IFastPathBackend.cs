// Device fast paths that the reference reaches only through `is VulkanBackend`
// casts.  With this interface those sites test `is IFastPathBackend` instead,
// so VulkanBackend and HipBackend both take them.  VulkanBackend already has
// every member below except TryRunModel with these signatures as internal
// methods; it implements the interface with one explicit forwarding line per
// member (and `=> false` for TryRunModel), e.g.
//   Tensor? IFastPathBackend.TryEndToEndTopK(Tensor i, int m, int c) => TryEndToEndTopK(i, m, c);
//
// Each site changes in one place: `X is VulkanBackend vulkan` (or
// `as VulkanBackend`) becomes `X is IFastPathBackend vulkan`; the call that
// follows is unchanged.
//
// NOT BUILT IN THIS REPOSITORY (no .NET SDK in the image); source for the
// reference's src/SimdYolo/.
namespace SimdYolo;

internal interface IFastPathBackend
{
    // PtModel.cs:533 (PT end-to-end head), VulkanTopK.cs:15.
    Tensor? TryEndToEndTopK(Tensor input, int maximum, int classes);
    // PtModel.cs:519 (Segment/Pose end-to-end head with extra rows), VulkanTopK.cs:18.
    Tensor? TryEndToEndTopKWithExtras(Tensor input, Tensor extras, int maximum, int classes);
    // OnnxEndToEnd.cs:152 (ONNX end-to-end export), VulkanTopK.cs:26.
    Tensor? TryEndToEndTopKOnnx(Tensor input, int maximum, int classes);
    // PtModel.cs:456,484-490 (joined multi-level head decode), VulkanExecution.cs:295.
    Tensor DecodeHeadLevels(DetectionHeadLevel[] levels, int[] shape, int bins, bool xyxy);
    // YoloDetector.cs:293-294 (replay of a recorded frame), VulkanReplay.cs:99.
    bool TryReplay(Tensor input, out Tensor[] outputs, CpuTensorPool? outputPool);
    // YoloDetector.cs:296 (start recording the frame that TryReplay may replay later).
    void BeginReplayCapture(Tensor input);
    // YoloDetector.cs:300 (one batched readback of the frame's outputs), VulkanDownloads.cs:14.
    void DownloadFrameOutputs(Tensor[] outputs, CpuTensorPool? outputPool);
    // YoloDetector.cs:182.
    long ReplayedFrames { get; }
    // YoloDetector.cs:291 (new site, before TryReplay): run the whole model natively when the backend has a
    // native forward for it (HipBackend: the library's sy_model_* walk for YOLOv8 / YOLO11 / YOLO26 PT
    // models).  VulkanBackend returns false.
    bool TryRunModel(object model, Tensor input, CpuTensorPool? outputPool, out Tensor[] outputs);
}
